"""Benchmark: accumulate_uz forward+backward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c4|c3|c2]
                    [--no-cpu-baseline]

A step is one accumulate_uz forward plus its backward (autograd into x and
the weights) over one batch of synthetic input already resident in HBM.
Default workload: BASELINE config 4's int64-stress shape, the largest
single-GPU accumulate_uz fwd+bwd configuration -- B=1, C=1, H=W=8192, R=6
half-plane (S=85), fp32, x the seeded piecewise-smooth image,
w = softplus(N(0,1)) times the forward box, upstream gradients N(0,1).

Prints ONE JSON line: metric/value in Mpixel-shifts/s (N*S per second,
whole job), the roofline of the backward pass (the dominant one: the
accumulate_uz_bwd_scatter_kernel launch plus its spill fix-up launch;
algorithmic HBM bytes over the pass's HIP-event-timed duration against the
8 TB/s peak, with the counter-measured bytes of the same kernel source from
profiles/) and the CPU baseline (the oracle's reference-order C
restatement timed on a bounded crop on this host's cores).
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "accumulate_uz fwd+bwd Mpixel-shifts/s; achieved HBM GB/s as % of MI355X peak"

CONFIGS = {
    # name: (B, C, H, W, R, table, dtype, comp_box)
    "c4": (1, 1, 8192, 8192, 6, "half", "float32", True),
    "c3": (16, 3, 256, 256, 5, "window", "float32", True),
    "c2": (4, 1, 512, 512, 7, "half", "float16", True),
}


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _kernel_source_hash() -> str:
    p = os.path.join(ROOT, "neural_shift_cuda_amd", "csrc", "accumulate.hip")
    return hashlib.sha256(open(p, "rb").read()).hexdigest()[:16]


def _traffic(config: str):
    """Measured HBM bytes per backward launch from a committed rocprofv3
    --pmc summary of this exact kernel source, else None."""
    p = os.path.join(ROOT, "profiles", f"accumulate_uz_bwd_{config}_traffic.json")
    try:
        d = json.load(open(p))
    except (OSError, ValueError):
        return None
    if d.get("kernel_source_sha256_16") != _kernel_source_hash():
        return None
    return d.get("hbm_bytes_per_launch")


def make_inputs(config: str, device):
    import torch
    from neural_shift_cuda_amd.workloads import (box_stack, halfplane_shifts, synthetic_image,
                                                 window_shifts)
    B, C, H, W, R, table, dt, comp_box = CONFIGS[config]
    dtype = getattr(torch, dt)
    sh = halfplane_shifts(R) if table == "half" else window_shifts(R)
    S = sh.size(0)
    x = synthetic_image(B, C, H, W, seed=1234).to(device=device, dtype=dtype)
    w = torch.empty(S * B, C, H, W, device=device, dtype=dtype)
    g = torch.Generator(device=device).manual_seed(4321)
    for s in range(S):  # plane by plane: no full-size temporaries
        blk = torch.nn.functional.softplus(
            torch.randn(B, C, H, W, generator=g, device=device, dtype=torch.float32))
        if comp_box:
            blk = blk * box_stack(sh[s:s + 1], 1, H, W, device=device)
        w[s * B:(s + 1) * B] = blk.to(dtype)
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    gU = torch.randn(B, C, H, W, generator=g, device=device, dtype=acc)
    gZ = torch.randn(B, C, H, W, generator=g, device=device, dtype=acc)
    return x, w, sh.to(device), gU, gZ


def cpu_baseline(config: str, budget_s: float = 10.0):
    """Oracle (reference-order C, OpenMP) fwd+bwd on a crop of the workload."""
    import torch

    import oracle
    from neural_shift_cuda_amd.workloads import box_stack, halfplane_shifts, window_shifts
    oracle.build()
    B, C, H, W, R, table, dt, comp_box = CONFIGS[config]
    ch, cw = min(H, 2048), min(W, 2048)
    Bc = 1
    sh = halfplane_shifts(R) if table == "half" else window_shifts(R)
    S = sh.size(0)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(Bc, C, ch, cw, generator=g)
    w = torch.nn.functional.softplus(torch.randn(S * Bc, C, ch, cw, generator=g))
    if comp_box:
        w = w * box_stack(sh, Bc, ch, cw)
    gU = torch.randn(Bc, C, ch, cw, generator=g)
    gZ = torch.randn(Bc, C, ch, cw, generator=g)
    units = Bc * C * ch * cw * S
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.accumulate_uz(x, w, sh, dtype=torch.float32)
        oracle.accumulate_uz_bwd(x, w, gU, gZ, sh, dtype=torch.float32)
        reps += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt_s = time.perf_counter() - t0
    return {
        "value": round(units * reps / dt_s / 1e6, 2),
        "unit": "Mpixel-shifts/s",
        "cores": oracle.max_threads(),
        "kind": "port",
        "sample": (f"oracle/oracle.c fp32 reference-order fwd+bwd on a {Bc}x{C}x{ch}x{cw} "
                   f"crop of {config} (S={S}), {reps} reps in {dt_s:.1f}s"),
    }


def copy_peak_gbs(device, nbytes: int = 4 << 30) -> float:
    import torch
    a = torch.empty(nbytes // 4, dtype=torch.float32, device=device)
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) / 5 / 1e3
    del a, b
    return 2 * nbytes / t / 1e9


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c4", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    a = ap.parse_args()

    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; multi-GPU runs are not part "
              "of it (the op shards by batch or by spatial band, see DESIGN.md)",
              file=sys.stderr)
        return 2

    import torch
    from neural_shift_cuda import accumulate_uz
    from neural_shift_cuda_amd import ops
    if not ops._HAS_CUDA_EXT:
        raise RuntimeError(f"HIP library failed to load: {ops._EXT_IMPORT_ERROR}")
    dev = torch.device("cuda:0")
    B, C, H, W, R, table, dt, comp_box = CONFIGS[a.config]

    _log(f"config {a.config}: generating inputs")
    x, w, sh, gU, gZ = make_inputs(a.config, dev)
    S = sh.size(0)
    N = B * C * H * W
    e = x.element_size()
    acc_b = gU.element_size()
    x.requires_grad_(True)
    w.requires_grad_(True)

    def step(ev=None):
        x.grad = None
        w.grad = None
        if ev:
            ev[0].record()
        U, Z = accumulate_uz(x, w, sh)
        if ev:
            ev[1].record()
        torch.autograd.backward([U, Z], [gU, gZ])
        if ev:
            ev[2].record()

    _log(f"warmup {a.warmup}")
    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()

    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(a.steps)]
    _log(f"timing {a.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(a.steps):
        step(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    fwd_ms = [ev[0].elapsed_time(ev[1]) for ev in evs]
    bwd_ms = [ev[1].elapsed_time(ev[2]) for ev in evs]
    ms_per_step = wall * 1e3 / a.steps

    units = N * S
    value = units / (ms_per_step / 1e3) / 1e6
    bytes_fwd = e * N * (S + 1) + 2 * acc_b * N
    bytes_bwd = 2 * e * N * (S + 1) + 2 * acc_b * N
    bwd_avg = statistics.mean(bwd_ms) / 1e3
    fwd_avg = statistics.mean(fwd_ms) / 1e3
    achieved = bytes_bwd / bwd_avg / 1e9
    step_gbs = (bytes_fwd + bytes_bwd) / (ms_per_step / 1e3) / 1e9
    _log(f"fwd {fwd_avg*1e3:.3f} ms ({bytes_fwd/fwd_avg/1e9:.0f} GB/s), "
         f"bwd {bwd_avg*1e3:.3f} ms ({achieved:.0f} GB/s), step {ms_per_step:.3f} ms")
    copy_gbs = copy_peak_gbs(dev)

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "Mpixel-shifts/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if dt == "float32" else ("f64" if dt == "float64" else f"{dt}->f32"),
        "data": "synthetic",
        "config": {
            "workload": f"accumulate_uz fwd+bwd {a.config}: B={B} C={C} H={H} W={W} R={R} "
                        f"{table} S={S} {dt} comp_box={comp_box}",
            "N": N, "S": S, "units_per_step": units,
        },
        "step_hbm_gbs": round(step_gbs, 1),
        "step_hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        "fwd_ms": round(fwd_avg * 1e3, 4),
        "bwd_ms": round(bwd_avg * 1e3, 4),
        "fwd_hbm_gbs": round(bytes_fwd / fwd_avg / 1e9, 1),
        "copy_peak_gbs": round(copy_gbs, 1),
        "roofline": {
            "kernel": "accumulate_uz backward pass: accumulate_uz_bwd_scatter_kernel + "
                      "accumulate_uz_spill_fixup_kernel",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": _traffic(a.config),
            "algorithmic_bytes_per_launch": bytes_bwd,
        },
    }
    del x, w, gU, gZ
    torch.cuda.empty_cache()
    if not a.no_cpu_baseline:
        _log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(a.config, a.cpu_budget)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

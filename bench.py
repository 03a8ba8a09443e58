"""Benchmark: accumulate_uz forward+backward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c4|c3|c2]
                    [--no-cpu-baseline]
    python bench.py --suite [--only OP ...]      every op at its BASELINE config
    python bench.py --cpu-suite                  the CPU baseline plan, no GPU
    python bench.py --mall-probe                 streaming probes, MALL reuse

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
profiles/), the streaming probes measured by the library's hand-written
probe kernels, and the CPU baseline (the reference's CPU path -- this
package's PyTorch fallback -- on a bounded sample of crops on every host
core, the oracle's C restatement beside it).
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


def cpu_model() -> str:
    """The host CPU's model name (lscpu, else /proc/cpuinfo), with the CPUID
    family/model/stepping from /proc/cpuinfo (a virtualised host may report
    only a generic name)."""
    import subprocess
    name = "unknown"
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.strip().startswith("Model name:"):
                name = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    ids = {}
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k == "model name" and name == "unknown":
                name = v.strip()
            if k in ("cpu family", "model", "stepping") and k not in ids:
                ids[k] = v.strip()
            if not line.strip() and ids:
                break
    except OSError:
        pass
    if ids:
        name += " (family %s model %s stepping %s)" % (
            ids.get("cpu family", "?"), ids.get("model", "?"), ids.get("stepping", "?"))
    return name


def _cpu_threads() -> int:
    """Use every host core for the CPU baselines."""
    import torch
    torch.set_num_threads(os.cpu_count() or 1)
    return torch.get_num_threads()


def _fallback_crop_inputs(config: str, ch: int, cw: int, seed: int):
    """(x, w, shifts, gU, gZ) of a ch x cw crop of `config` on the CPU, in
    the configuration's dtype (the fallback promotes like the reference)."""
    import torch
    from neural_shift_cuda_amd.workloads import (box_stack, halfplane_shifts, softplus_weights,
                                                 synthetic_image, window_shifts)
    B, C, H, W, R, table, dt, comp_box = CONFIGS[config]
    dtype = getattr(torch, dt)
    sh = halfplane_shifts(R) if table == "half" else window_shifts(R)
    S = sh.size(0)
    x = synthetic_image(1, C, ch, cw, seed=seed)
    w = softplus_weights((S, C, ch, cw), seed=seed + 1)
    if comp_box:
        w = w * box_stack(sh, 1, ch, cw)
    g = torch.Generator().manual_seed(seed + 2)
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    gU = torch.randn(1, C, ch, cw, generator=g, dtype=acc)
    gZ = torch.randn(1, C, ch, cw, generator=g, dtype=acc)
    return x.to(dtype), w.to(dtype), sh, gU, gZ


def cpu_baseline(config: str, budget_s: float = 15.0):
    """The reference's CPU path on a bounded sample of the workload: the
    package's PyTorch fallback (accumulate_uz_reference, bit-exact with the
    reference's own fallback on the golden vectors) forward plus autograd
    backward on 256 x 256 crops of `config`, timed with perf_counter on all
    host cores until `budget_s` is spent.  The oracle's C restatement
    (OpenMP) on the same crops is reported beside it."""
    import torch

    import oracle
    from neural_shift_cuda import accumulate_uz
    threads = _cpu_threads()
    ch = cw = 256
    crops, units, t_fb, k = 0, 0, 0.0, 0
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or crops < 2:
        x, w, sh, gU, gZ = _fallback_crop_inputs(config, ch, cw, 900 + k)
        k += 1
        xr, wr = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
        t0 = time.perf_counter()
        U, Z = accumulate_uz(xr, wr, sh)
        torch.autograd.backward([U, Z], [gU, gZ])
        t_fb += time.perf_counter() - t0
        crops += 1
        units += x.numel() * sh.size(0)
    oracle.build()
    t0 = time.perf_counter()
    reps = 0
    while reps < 2 or time.perf_counter() - t0 < budget_s / 3:
        oracle.accumulate_uz(x, w, sh, dtype=torch.float32)
        oracle.accumulate_uz_bwd(x, w, gU, gZ, sh, dtype=torch.float32)
        reps += 1
    t_or = time.perf_counter() - t0
    per_crop = x.numel() * sh.size(0)
    return {
        "value": round(units / t_fb / 1e6, 2),
        "unit": "Mpixel-shifts/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"package PyTorch CPU fallback (accumulate_uz_reference fwd + autograd bwd, "
                   f"bit-exact with the reference fallback), {crops} crops of 1x1x{ch}x{cw} "
                   f"of {config} (S={sh.size(0)}) in {t_fb:.1f}s; rate per pixel-shift, "
                   f"extrapolated to the full workload"),
        "cpu_model": cpu_model(),
        "oracle_c": {"value": round(per_crop * reps / t_or / 1e6, 2),
                     "cores": oracle.max_threads(),
                     "sample": f"oracle/oracle.c fp32 fwd+bwd, {reps} reps of one crop"},
    }


def stream_probes(device, nbytes: int = 4 << 30, reps: int = 3) -> dict:
    """Measured streaming rates of this GPU, GB/s: the hand-written probe
    kernels of the library (nsh_stream_probe: 16-byte accesses) reading,
    copying and filling a `nbytes` buffer.  Each kind is the best over its
    variants -- 4, 8 or 16 loads in flight per lane, workgroups of 256 or
    1024 lanes, 1 to 32 per CU, temporal or streaming loads and stores
    (copy, fill), bursts or a per-lane prefetch ring (copy) -- of the best of
    `reps` launches each (HIP events
    on the launch stream); the winning variant is reported beside it.  A
    copy moves 2 * nbytes."""
    import itertools
    import torch
    from neural_shift_cuda_amd import _C
    a = torch.empty(nbytes // 4, dtype=torch.float32, device=device)
    b = torch.empty_like(a)
    _C.stream_probe("fill", None, a)
    _C.stream_probe("fill", None, b)
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    out, won = {}, {}
    for kind, moved in (("read", nbytes), ("read_nt", nbytes), ("copy", 2 * nbytes),
                        ("fill", nbytes)):
        src = a if kind != "fill" else None
        best, best_v = float("inf"), None
        plain_l = (False, True) if kind == "copy" else (False,)
        plain_s = (False, True) if kind in ("copy", "fill") else (False,)
        rings = (False, True) if kind == "copy" else (False,)
        for unroll, lanes, per_cu, pl, ps, rg in itertools.product(
                (4, 8, 16), (256, 1024), (1, 2, 4, 8, 16, 32), plain_l, plain_s, rings):
            wg = per_cu * cus * 256 // lanes
            if wg < cus:
                continue
            kw = dict(unroll=unroll, lanes=lanes, plain_loads=pl, plain_stores=ps, ring=rg)
            _C.stream_probe(kind, src, b, wg, **kw)
            for _ in range(reps):
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record()
                _C.stream_probe(kind, src, b, wg, **kw)
                e1.record()
                e1.synchronize()
                t = e0.elapsed_time(e1) / 1e3
                if t < best:
                    best = t
                    best_v = (f"unroll {unroll}, {lanes} lanes x {wg} workgroups"
                              + (", prefetch ring" if rg else "")
                              + (", temporal loads" if pl else "")
                              + (", temporal stores" if ps else ""))
        out[f"{kind}_gbs"] = round(moved / best / 1e9, 1)
        won[kind] = best_v
    out["variants"] = won
    del a, b
    torch.cuda.empty_cache()
    return out


def mall_probe(device, sizes_mb=(32, 64, 128, 192, 256, 320, 384, 512, 1024), reps: int = 5):
    """Does a second read of a just-read buffer come from the 256 MB
    Infinity Cache (MALL)?  For each size: evict (read 2 GiB of another
    buffer), then time a first and an immediately following second read of
    the same buffer with the probe's read kernel; best of `reps`."""
    import torch
    from neural_shift_cuda_amd import _C
    big = torch.empty(max(sizes_mb) << 20, dtype=torch.uint8, device=device)
    other = torch.empty(2 << 30, dtype=torch.uint8, device=device)
    sink = torch.empty(4096, dtype=torch.uint8, device=device)
    _C.stream_probe("fill", None, big)
    _C.stream_probe("fill", None, other)
    rows = []
    for mb in sizes_mb:
        buf = big[: mb << 20]
        t1 = t2 = float("inf")
        for _ in range(reps):
            _C.stream_probe("read", other, sink)
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
            ev[0].record()
            _C.stream_probe("read", buf, sink)
            ev[1].record()
            _C.stream_probe("read", buf, sink)
            ev[2].record()
            ev[2].synchronize()
            t1 = min(t1, ev[0].elapsed_time(ev[1]) / 1e3)
            t2 = min(t2, ev[1].elapsed_time(ev[2]) / 1e3)
        rows.append({"mb": mb, "first_read_gbs": round((mb << 20) / t1 / 1e9, 1),
                     "second_read_gbs": round((mb << 20) / t2 / 1e9, 1)})
    del big, other, sink
    torch.cuda.empty_cache()
    return rows


def _time_calls(fn, steps: int, warmup: int) -> float:
    """Mean duration in ms of `fn()` over `steps` calls, each bracketed by HIP
    events on torch's current stream (the stream the kernels are launched on)."""
    import torch
    out = None
    for _ in range(warmup):
        out = fn()
    del out
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    keep = []
    for e0, e1 in evs:
        e0.record()
        keep.append(fn())
        e1.record()
        if len(keep) > 1:
            keep.pop(0)
    torch.cuda.synchronize()
    return statistics.mean(e0.elapsed_time(e1) for e0, e1 in evs)


def suite(dev, steps: int, warmup: int, only=None):
    """Every op of the path at its BASELINE configuration, one pass at a time,
    through the C-ABI wrappers (`_C`): yields one dict per (op, config, pass)
    with the HIP-event time and the algorithmic HBM bytes of that pass.

    Algorithmic bytes (each tensor at the API boundary touched once; e = user
    element bytes, a = accumulator bytes, N = B*C*H*W, S = shift rows):
      accumulate_uz      fwd e*N*(S+1) + 2a*N        bwd 2e*N*(S+1) + 2a*N
      normalized         fwd e*N*(S+1) + 2a*N        bwd 2e*N*(S+1) + 4a*N
      shift_gather       fwd e*N*(1+S) + e*S*B*H*W   bwd e*N*S + e*N
      pair_gather        fwd e*N + 2e*S*N + e*S*B*H*W bwd 2e*N*S + e*N
      metropolis (fused) fwd e*N*(S+1) + 2e*N  (single read of w_half; the
                         two-pass kernel pair reads it twice)
                         bwd 2e*N*S + 5e*N + a*N (w_half read and grad_w_half
                         written once; img, grad_Wx, grad_d_hat, d_hat and the
                         degree read, grad_img written)
      scalar             fwd e*N + 2a*N + e*S*B*C    bwd e*N + 2a*N + e*N + e*S*B*C
      normalized, shared weights (P = S*B*H*W shared weight elements):
                         fwd e*P + e*N + 2a*N        bwd e*P + e*S*N + e*N + 4a*N
                         (the weight gradient is written per channel);
                         the broadcast-copy form adds the copy (read P, write
                         S*N) and reads S*N weights instead of P
    """
    import torch
    from neural_shift_cuda_amd import _C
    from neural_shift_cuda_amd.workloads import (box_stack, halfplane_shifts, logit_weights,
                                                 synthetic_image, window_shifts)

    def want(name):
        return only is None or name in only

    def rec(op, cfg, pas, ms, nbytes, units, dtype, extra=None):
        d = {"op": op, "config": cfg, "pass": pas, "ms": round(ms, 4),
             "alg_bytes": int(nbytes), "gbs": round(nbytes / ms / 1e6, 1),
             "hbm_frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
             "units": int(units), "mpix_shifts_s": round(units / ms / 1e3, 1),
             "dtype": dtype}
        if extra:
            d.update(extra)
        _log(f"suite {op} {cfg} {pas}: {ms:.4f} ms, {d['gbs']} GB/s ({100*d['hbm_frac']:.1f}%)")
        return d

    def weights(sh, B, C, H, W, seed, dtype, comp_box):
        g = torch.Generator(device=dev).manual_seed(seed)
        S = sh.size(0)
        w = torch.empty(S * B, C, H, W, device=dev, dtype=dtype)
        for s in range(S):
            blk = torch.nn.functional.softplus(
                torch.randn(B, C, H, W, generator=g, device=dev, dtype=torch.float32))
            if comp_box:
                blk = blk * box_stack(sh[s:s + 1], 1, H, W, device=dev)
            w[s * B:(s + 1) * B] = blk.to(dtype)
        return w

    def acc_pair(op, cfg, B, C, H, W, sh, dtype, w, normalized=False, log_w=False, codes=False,
                 band=None):
        x = synthetic_image(B, C, H, W, seed=11).to(device=dev, dtype=dtype)
        acc = torch.float64 if dtype == torch.float64 else torch.float32
        g = torch.Generator(device=dev).manual_seed(12)
        g1 = torch.randn(B, C, H, W, generator=g, device=dev, dtype=acc)
        g2 = torch.randn(B, C, H, W, generator=g, device=dev, dtype=acc)
        S = sh.size(0)
        N = B * C * H * W
        e, a = x.element_size(), g1.element_size()
        shd = sh.to(dev)
        dn = str(dtype).replace("torch.", "")
        if normalized:
            D, L = _C.normalized_accumulate_uz_forward(x, w, shd, log_w, row_codes=codes)
            f = _time_calls(lambda: _C.normalized_accumulate_uz_forward(
                x, w, shd, log_w, row_codes=codes), steps, warmup)
            b = _time_calls(lambda: _C.normalized_accumulate_uz_backward(
                x, w, D, L, g1, g2, shd, log_w, row_codes=codes), steps, warmup)
            bb = 2 * e * N * (S + 1) + 4 * a * N
        else:
            f = _time_calls(lambda: _C.accumulate_uz_forward(x, w, shd, row_codes=codes,
                                                             band=band), steps, warmup)
            b = _time_calls(lambda: _C.accumulate_uz_backward(x, w, g1, g2, shd, row_codes=codes,
                                                              band=band), steps, warmup)
            bb = 2 * e * N * (S + 1) + 2 * a * N
        fb = e * N * (S + 1) + 2 * a * N
        return [rec(op, cfg, "fwd", f, fb, N * S, dn), rec(op, cfg, "bwd", b, bb, N * S, dn)]

    out = []
    # c1: gathers, bf16, B=8 C=3 256^2; box = half-plane R=5 (61 rows), periodic = 121 rows
    for mode, sh in (("box", halfplane_shifts(5)), ("periodic", window_shifts(5))):
        B, C, H, W = 8, 3, 256, 256
        g = synthetic_image(B, C, H, W, seed=21).to(device=dev, dtype=torch.bfloat16)
        shd = sh.to(dev)
        S, N, e = sh.size(0), B * C * H * W, 2
        for op, fwd, bwdf, pair in (
                ("shift_gather", _C.shift_gather_forward, _C.shift_gather_backward, False),
                ("pair_gather", _C.pair_gather_forward, _C.pair_gather_backward, True)):
            if not want(op):
                continue
            f = _time_calls(lambda: fwd(g, shd), steps, warmup)
            go = torch.randn(S * B, 2 * C if pair else C, H, W, device=dev).to(torch.bfloat16)
            b = _time_calls(lambda: bwdf(go, shd, B, C, H, W), steps, warmup)
            fb = (e * N + 2 * e * S * N if pair else e * N * (1 + S)) + e * S * B * H * W
            bb = (2 if pair else 1) * e * N * S + e * N
            out += [rec(op, f"c1 {mode}", "fwd", f, fb, N * S, "bf16"),
                    rec(op, f"c1 {mode}", "bwd", b, bb, N * S, "bf16")]
            del go
    # c0: the reference's CPU-runnable case, fp32 1x1x256^2, R=3 half-plane
    # (S=25), comp_box softplus weights
    if want("accumulate_uz"):
        sh0 = halfplane_shifts(3)
        w = weights(sh0, 1, 1, 256, 256, 21, torch.float32, True)
        out += acc_pair("accumulate_uz", "c0", 1, 1, 256, 256, sh0, torch.float32, w)
        del w
    # c2: fp16 B=4 C=1 512^2 R=7 half-plane (S=113)
    B, C, H, W = 4, 1, 512, 512
    sh = halfplane_shifts(7)
    if want("accumulate_uz"):
        w = weights(sh, B, C, H, W, 31, torch.float16, True)
        out += acc_pair("accumulate_uz", "c2", B, C, H, W, sh, torch.float16, w)
        del w
    if want("normalized_accumulate_uz"):
        lw = logit_weights((sh.size(0) * B, C, H, W), seed=32, device=dev).to(torch.float16)
        out += acc_pair("normalized_accumulate_uz", "c2 log", B, C, H, W, sh, torch.float16, lw,
                        normalized=True, log_w=True)
        # the same logits in fp32 (not a BASELINE configuration): separates
        # the cost of the log-weight arithmetic from that of the 16-bit type
        out += acc_pair("normalized_accumulate_uz", "c2 shape, fp32 logits", B, C, H, W, sh,
                        torch.float32, lw.float(), normalized=True, log_w=True)
        del lw
    # c3: GASD full window R=5 (121 rows), fp32 B=16 C=3 256^2; fp64 at B=2
    sh = window_shifts(5)
    for dtype, B in ((torch.float32, 16), (torch.float64, 2)):
        C, H, W = 3, 256, 256
        tag = "c3" if dtype == torch.float32 else "c3 fp64"
        if not (want("accumulate_uz") or want("normalized_accumulate_uz")):
            break
        w = weights(sh, B, C, H, W, 41, dtype, True)
        if want("accumulate_uz"):
            out += acc_pair("accumulate_uz", tag, B, C, H, W, sh, dtype, w)
        if want("normalized_accumulate_uz"):
            out += acc_pair("normalized_accumulate_uz", tag + " pos", B, C, H, W, sh, dtype, w,
                            normalized=True)
        del w
    # c4: the headline shape, fp32 8192^2 R=6 half-plane (S=85), comp_box
    if want("accumulate_uz"):
        B, C, H, W = 1, 1, 8192, 8192
        sh4 = halfplane_shifts(6)
        w = weights(sh4, B, C, H, W, 51, torch.float32, True)
        out += acc_pair("accumulate_uz", "c4", B, C, H, W, sh4, torch.float32, w)
        del w
        torch.cuda.empty_cache()
    # table radius: the half-plane at R = 6 (c4's table), 8 (the LDS halo),
    # 10, 15 and 22 (S = 1013, the top of the reference's 1 <= S <= 1024) and
    # the full window at R = 15 (S = 961), fp32 comp_box weights on one
    # 4096^2 image (the R = 22 weights and their gradient are 68 GB each)
    if want("accumulate_uz_radius"):
        B, C, H, W = 1, 1, 4096, 4096
        for name, shr in (("half R=6", halfplane_shifts(6)), ("half R=8", halfplane_shifts(8)),
                          ("half R=10", halfplane_shifts(10)),
                          ("half R=15", halfplane_shifts(15)),
                          ("half R=22", halfplane_shifts(22)),
                          ("window R=15", window_shifts(15))):
            w = weights(shr, B, C, H, W, 53, torch.float32, True)
            out += acc_pair("accumulate_uz_radius", f"{H}x{W} {name} S={shr.size(0)}", B, C, H,
                            W, shr, torch.float32, w)
            del w
            torch.cuda.empty_cache()
    # one GPU's share of c4 split into 8 horizontal bands: 1024 rows plus the
    # R = 6 halo rows on each side (the rows the neighbouring GPUs own), the
    # whole 8192 columns, through the band entry points (the band's place in
    # the image for the box tests; here the band of image rows 3072..4095);
    # the band's own 1024 rows are what that GPU keeps
    if want("accumulate_uz_band"):
        B, C, H, W = 1, 1, 8192 // 8 + 2 * 6, 8192
        sh4 = halfplane_shifts(6)
        w = weights(sh4, B, C, H, W, 52, torch.float32, True)
        out += acc_pair("accumulate_uz_band", "c4 1/8 band (1036x8192)", B, C, H, W, sh4,
                        torch.float32, w, band=(3 * 1024 - 6, 8192))
        del w
        torch.cuda.empty_cache()
    # single-head weights shared by the C = 3 channels (NeKDe/GASD with one
    # head), c3 image shape with the R = 5 half-plane: the kernels reading
    # the shared plane (shared_weights) against the reference installers'
    # broadcast copy (expand + contiguous, then the per-channel op) -- the
    # copy pass the shared form saves is inside the timed call
    if want("shared_weights"):
        B, C, H, W = 16, 3, 256, 256
        sh = halfplane_shifts(5)
        S, N = sh.size(0), B * C * H * W
        x = synthetic_image(B, C, H, W, seed=61).to(dev)
        w1 = weights(sh, B, 1, H, W, 62, torch.float32, False)
        shd = sh.to(dev)
        g = torch.Generator(device=dev).manual_seed(63)
        gD = torch.randn(B, C, H, W, generator=g, device=dev)
        gL = torch.randn(B, C, H, W, generator=g, device=dev)

        def bcast():
            return w1.expand(-1, C, -1, -1).contiguous()

        planes1 = S * B * H * W
        shared_fwd = 4 * planes1 + 4 * N + 8 * N
        mat_fwd = 4 * planes1 + 2 * 4 * S * N + 4 * N + 8 * N
        for mode in ("shared", "broadcast copy"):
            if mode == "shared":
                fwd = lambda: _C.normalized_accumulate_uz_forward(x, w1, shd, False,
                                                                  shared_weights=True)
                D, L = fwd()
                bwd = lambda: _C.normalized_accumulate_uz_backward(
                    x, w1, D, L, gD, gL, shd, False, shared_weights=True)
                fb, bb = shared_fwd, 4 * planes1 + 4 * S * N + 8 * N + 16 * N
            else:
                fwd = lambda: _C.normalized_accumulate_uz_forward(x, bcast(), shd, False)
                D, L = fwd()
                bwd = lambda: _C.normalized_accumulate_uz_backward(x, bcast(), D, L, gD, gL,
                                                                   shd, False)
                fb, bb = mat_fwd, 4 * planes1 + 3 * 4 * S * N + 8 * N + 16 * N
            f = _time_calls(fwd, steps, warmup)
            b = _time_calls(bwd, steps, warmup)
            out += [rec("normalized_shared_weights", f"c3 shape C=3 one head, {mode}", "fwd",
                        f, fb, N * S, "float32"),
                    rec("normalized_shared_weights", f"c3 shape C=3 one head, {mode}", "bwd",
                        b, bb, N * S, "float32")]
        del x, w1, gD, gL
    # two heads mixed to the C = 3 channels by a (C, h) matrix (NeKDe/GASD
    # inference), c3 image shape with the R = 5 half-plane and the forward
    # box in the kernels: the mixing product in the forward kernel's weight
    # load (normalized_accumulate_uz_mixed: each channel reads its h head
    # planes) against mixing first (the mixing kernel writing the (S*B, C,
    # H, W) stack, then the plain forward); the mixing pass is inside the
    # timed call.  Both rows quote the op's boundary bytes (head planes, x and the
    # outputs once: 4*h*P + 12*N); the fused kernel reads C*h*P, the
    # mixed-first pair h*P + 2*C*P (P = S*B*H*W)
    if want("head_mix"):
        from neural_shift_cuda_amd.ops import _mirror_table
        B, C, H, W, h = 16, 3, 256, 256, 2
        sh = halfplane_shifts(5)
        S, N = sh.size(0), B * C * H * W
        P = S * B * H * W
        x = synthetic_image(B, C, H, W, seed=71).to(dev)
        hw = weights(sh, B, h, H, W, 72, torch.float32, False)
        g = torch.Generator(device=dev).manual_seed(73)
        mix = torch.softmax(torch.randn(C, h, generator=g, device=dev), dim=1)
        table, codes = _mirror_table(sh.to(dev), False, True)
        served = _C.normalized_accumulate_uz_forward_mixed(x, hw, mix, table, row_codes=codes)
        assert served is not None, "head_mix row: the fused entry point must serve c3"

        def mixed_first():
            m = _C.head_mix_forward(hw.reshape(S * B, h, H * W), mix).view(S * B, C, H, W)
            return _C.normalized_accumulate_uz_forward(x, m, table, False, row_codes=codes)

        fb = 4 * h * P + 12 * N
        f = _time_calls(lambda: _C.normalized_accumulate_uz_forward_mixed(
            x, hw, mix, table, row_codes=codes), steps, warmup)
        u = _time_calls(mixed_first, steps, warmup)
        out += [rec("normalized_head_mix", "c3 shape C=3 two heads, box, fused", "fwd", f, fb,
                    N * S, "float32", {"kernel_bytes": 4 * C * h * P + 12 * N}),
                rec("normalized_head_mix", "c3 shape C=3 two heads, box, mixed first", "fwd",
                    u, fb, N * S, "float32", {"kernel_bytes": 4 * (h + 2 * C) * P + 12 * N})]
        # the training path's mixing product alone (autograd through it):
        # the HIP kernels (nsh_head_mix_forward / _backward) against the
        # reference installers' einsum and its autograd backward; bytes: the
        # forward reads h and writes C planes, the backward reads C + h and
        # writes h planes (the matrix gradient is a reduction)
        wt = hw.reshape(S * B, h, H * W)
        gout = torch.randn(S * B, C, H * W, generator=g, device=dev)
        wq = wt.detach().requires_grad_(True)
        mq = mix.detach().requires_grad_(True)

        def einsum_bwd():
            o = torch.einsum("ch,nhp->ncp", mq, wq)
            return torch.autograd.grad(o, (wq, mq), gout)

        kf = _time_calls(lambda: _C.head_mix_forward(wt, mix), steps, warmup)
        kb = _time_calls(lambda: _C.head_mix_backward(wt, mix, gout), steps, warmup)
        ef = _time_calls(lambda: torch.einsum("ch,nhp->ncp", mix, wt), steps, warmup)
        eb = _time_calls(einsum_bwd, steps, warmup)  # forward + backward
        mfb, mbb = 4 * (h + C) * P, 4 * (C + 2 * h) * P
        out += [rec("head_mix", "c3 shape C=3 two heads, kernels", "fwd", kf, mfb, P, "float32"),
                rec("head_mix", "c3 shape C=3 two heads, kernels", "bwd", kb, mbb, P, "float32"),
                rec("head_mix", "c3 shape C=3 two heads, reference einsum", "fwd", ef, mfb, P,
                    "float32"),
                rec("head_mix", "c3 shape C=3 two heads, reference einsum", "fwd+bwd", eb,
                    mfb + mbb, P, "float32")]
        del x, hw, served, wt, gout, wq, mq
    # scalar (GADSD), c3 shape fp32, 121 transforms
    if want("accumulate_uz_scalar"):
        B, C, H, W = 16, 3, 256, 256
        sh = window_shifts(5)
        S, N = sh.size(0), B * C * H * W
        x = synthetic_image(B, C, H, W, seed=51).to(dev)
        ws = torch.rand(S, B, C, device=dev)
        shd = sh.to(dev)
        gU = torch.randn(B, C, H, W, device=dev)
        gZ = torch.randn(B, C, H, W, device=dev)
        f = _time_calls(lambda: _C.accumulate_uz_scalar_forward(x, ws, shd), steps, warmup)
        b = _time_calls(lambda: _C.accumulate_uz_scalar_backward(x, ws, gU, gZ, shd), steps,
                        warmup)
        out += [rec("accumulate_uz_scalar", "c3 shape", "fwd", f, 4 * N + 8 * N + 4 * S * B * C,
                    N * S, "float32"),
                rec("accumulate_uz_scalar", "c3 shape", "bwd", b,
                    4 * N + 8 * N + 4 * N + 4 * S * B * C, N * S, "float32")]
        del x, gU, gZ
    # periodic half-plane at the c4 shape: circular mirrors (S = 85 rows,
    # row code 2) against the explicit mirror rows the reference's
    # installers build (169 rows, rolled weight planes)
    if want("accumulate_uz_periodic"):
        B, C, H, W = 1, 1, 8192, 8192
        sh = halfplane_shifts(6)
        w = weights(sh, B, C, H, W, 41, torch.float32, False)
        circ = sh.clone()
        circ[:, 2] *= 2
        out += acc_pair("accumulate_uz_periodic", "c4 circular mirrors", B, C, H, W, circ,
                        torch.float32, w, codes=True)
        rows, planes = [], []
        for s_, (dx, dy, inv) in enumerate(sh.tolist()):
            rows.append((dx, dy, 0))
            planes.append(w[s_ * B:(s_ + 1) * B])
            if inv:
                rows.append((-dx, -dy, 0))
                planes.append(torch.roll(w[s_ * B:(s_ + 1) * B], shifts=(dx, dy), dims=(-2, -1)))
        we = torch.cat(planes)
        del planes, w
        out += acc_pair("accumulate_uz_periodic", "c4 explicit mirror rows", B, C, H, W,
                        torch.tensor(rows, dtype=torch.int64), torch.float32, we)
        del we
        torch.cuda.empty_cache()
    # c4: Metropolis fp32 8192^2 R=6 (S=85), use_box
    if want("metropolis_aggregate"):
        B, C, H, W = 1, 1, 8192, 8192
        sh = halfplane_shifts(6)
        S, N = sh.size(0), B * C * H * W
        wh = weights(sh, B, C, H, W, 61, torch.float32, False).view(B, S, C, H, W)
        img = synthetic_image(B, C, H, W, seed=62).to(dev)
        shd = sh.to(dev)
        f = _time_calls(lambda: _C.metropolis_aggregate(wh, img, shd, 1, 1e-6), steps, warmup)
        out.append(rec("metropolis_aggregate", "c4", "fwd", f, 4 * N * (S + 1) + 8 * N, N * S,
                       "float32", {"two_pass_bytes": 8 * N * S + 4 * N * 2 + 8 * N + 4 * N}))
        _, dh, deg = _C.metropolis_aggregate_with_degree(wh, img, shd, 1, 1e-6)
        gWx = torch.randn(B, C, H, W, device=dev)
        gdh = torch.randn(B, C, H, W, device=dev)
        b = _time_calls(lambda: _C.metropolis_aggregate_backward(wh, img, shd, 1, 1e-6, deg, dh,
                                                                 gWx, gdh), steps, warmup)
        out.append(rec("metropolis_aggregate", "c4", "bwd", b, 8 * N * S + 24 * N, N * S,
                       "float32"))
        del wh, img, dh, deg, gWx, gdh
    torch.cuda.empty_cache()
    return out


def summarize_traffic(prof_dir: str, config: str = "c4") -> dict:
    """HBM bytes per launch of the accumulate_uz passes from two rocprofv3
    counter runs of this script (`--pmc FETCH_SIZE`, then `--pmc WRITE_SIZE`,
    each with `--kernel-trace --output-format csv -o run` under
    prof_dir/pmc_<COUNTER>/).  The counters are calibrated on the input
    generator's plane copies (__amd_rocclr_copyBuffer of one H*W fp32 plane:
    known bytes read and written); an optional third run of the L2-to-fabric
    read-request counters by size (pmc_RDREQ/) cross-checks the read
    calibration.  Writes profiles/accumulate_uz_bwd_<config>_traffic.json
    keyed by the kernel source hash and returns it."""
    import csv
    import collections
    B, C, H, W = CONFIGS[config][:4]
    plane = B * C * H * W * 4
    per = {}
    scale = {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        path = os.path.join(prof_dir, f"pmc_{ctr}", "run_counter_collection.csv")
        vals = collections.defaultdict(list)
        copies = []
        for r in csv.DictReader(open(path)):
            n, v = r["Kernel_Name"], float(r["Counter_Value"]) * 1024.0
            if "copyBuffer" in n:
                copies.append(v)
            elif "nsh::accumulate_uz" in n or "nsh::spill_fixup" in n:
                vals[n.split("<")[0].replace("void nsh::", "") + "<" + n.split("<")[1].split(">")[0]
                     + ">"].append(v)
        ref = statistics.median(copies)
        scale[ctr] = plane / ref  # bytes the copy moved in that direction / counter bytes
        per[ctr] = {k: statistics.mean(v) * scale[ctr] for k, v in vals.items()}
    # Cross-check of the FETCH_SIZE calibration (optional third run under
    # prof_dir/pmc_RDREQ/ with --pmc TCC_EA0_RDREQ_32B_sum TCC_EA0_RDREQ_64B_sum
    # TCC_EA0_RDREQ_128B_sum TCC_EA0_RDREQ_sum): read bytes as request counts
    # times request sizes, which needs no calibration.
    rdreq = {}
    rq = os.path.join(prof_dir, "pmc_RDREQ", "run_counter_collection.csv")
    if os.path.exists(rq):
        acc = collections.defaultdict(lambda: collections.defaultdict(float))
        for r in csv.DictReader(open(rq)):
            n = r["Kernel_Name"]
            if "nsh::accumulate_uz" in n or "nsh::spill_fixup" in n:
                k = n.split("<")[0].replace("void nsh::", "") + "<" + n.split("<")[1].split(">")[0] + ">"
                acc[k][(r["Dispatch_Id"], r["Counter_Name"])] += float(r["Counter_Value"])
        for k, m in acc.items():
            tot = collections.defaultdict(list)
            for (_, c), v in m.items():
                tot[c].append(v)
            c = {n: statistics.mean(v) for n, v in tot.items()}
            sized = sum(c.get(f"TCC_EA0_RDREQ_{b}B_sum", 0.0) for b in (32, 64, 128))
            rdreq[k] = {
                "read_bytes": int(sum(b * c.get(f"TCC_EA0_RDREQ_{b}B_sum", 0.0)
                                      for b in (32, 64, 128))),
                "requests_sized_fraction": round(sized / c["TCC_EA0_RDREQ_sum"], 4)
                if c.get("TCC_EA0_RDREQ_sum") else None,
                "fetch_size_calibrated_ratio": round(
                    sum(b * c.get(f"TCC_EA0_RDREQ_{b}B_sum", 0.0) for b in (32, 64, 128))
                    / per["FETCH_SIZE"][k], 4) if per["FETCH_SIZE"].get(k) else None,
            }
    fwd = {k: per["FETCH_SIZE"][k] + per["WRITE_SIZE"][k] for k in per["FETCH_SIZE"]
           if "fwd" in k or "fixup_kernel<float, float, 2" in k}
    bwd = {k: per["FETCH_SIZE"][k] + per["WRITE_SIZE"][k] for k in per["FETCH_SIZE"]
           if "bwd" in k or "fixup_kernel<float, float, 1" in k}
    d = {
        "kernel": "accumulate_uz backward pass (accumulate_uz_bwd_scatter_kernel + "
                  "spill_fixup_kernel)",
        "config": config,
        "kernel_source_sha256_16": _kernel_source_hash(),
        "hbm_bytes_per_launch": int(sum(bwd.values())),
        "fwd_hbm_bytes_per_launch": int(sum(fwd.values())),
        "per_kernel_read_bytes": {k: int(v) for k, v in per["FETCH_SIZE"].items()},
        "per_kernel_write_bytes": {k: int(v) for k, v in per["WRITE_SIZE"].items()},
        "read_bytes_from_request_sizes": rdreq or None,
        "calibration": {"fetch_scale": round(scale["FETCH_SIZE"], 4),
                        "write_scale": round(scale["WRITE_SIZE"], 4),
                        "note": "bytes = counter KiB * 1024 * scale; scale from the "
                                "__amd_rocclr_copyBuffer plane copies of known size"},
    }
    out = os.path.join(ROOT, "profiles", f"accumulate_uz_bwd_{config}_traffic.json")
    with open(out, "w") as f:
        json.dump(d, f, indent=1)
        f.write("\n")
    return d


# rocprofv3 base counters of the --summarize-counters pass (8 SQ + 1 GRBM
# counters: one hardware pass on gfx950).
COUNTERS = ("SQ_WAVES SQ_INSTS_VALU SQ_ACTIVE_INST_VALU SQ_THREAD_CYCLES_VALU SQ_INSTS_LDS "
            "SQ_LDS_BANK_CONFLICT SQ_ACTIVE_INST_LDS SQ_BUSY_CU_CYCLES GRBM_GUI_ACTIVE")


def summarize_counters(raw_dir: str, cu_num: int = 256, xcc: int = 8) -> str:
    """Per-kernel VALU and LDS metrics (nsh kernels) from one rocprofv3
    `--pmc <COUNTERS> --kernel-trace --output-format csv -o run` pass under
    raw_dir.  Counter values of one dispatch are summed over their rows and
    averaged over the kernel's dispatches.  GRBM_GUI_ACTIVE is summed over
    the `xcc` XCDs, so it is divided by `xcc` to give the per-XCD busy cycles
    that rocprofv3's derived metrics reduce with max.  Formulas (rocprofv3
    derived metrics): VALUBusy = 100*SQ_ACTIVE_INST_VALU/CU_NUM/GUI_ACTIVE,
    VALUUtilization = 100*SQ_THREAD_CYCLES_VALU/(SQ_ACTIVE_INST_VALU*64),
    LDSBankConflict = 100*SQ_LDS_BANK_CONFLICT/GUI_ACTIVE/CU_NUM."""
    import collections
    import csv
    csv.field_size_limit(1 << 30)
    vals = collections.defaultdict(lambda: collections.defaultdict(float))
    dur = collections.defaultdict(dict)
    for r in csv.DictReader(open(os.path.join(raw_dir, "run_counter_collection.csv"))):
        n = r["Kernel_Name"]
        if "nsh::" not in n and not n.startswith("_ZN3nsh"):  # 16-bit kernels stay mangled
            continue
        k = n.replace("void nsh::", "").split("(")[0]
        d = r["Dispatch_Id"]
        vals[k][(d, r["Counter_Name"])] += float(r["Counter_Value"])
        dur[k][d] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    rows = []
    for k, m in vals.items():
        per = collections.defaultdict(list)
        for (_, c), v in m.items():
            per[c].append(v)
        c = {n: sum(v) / len(v) for n, v in per.items()}
        gui = c["GRBM_GUI_ACTIVE"] / xcc
        act = c["SQ_ACTIVE_INST_VALU"]
        rows.append((k, len(dur[k]), sum(dur[k].values()) / len(dur[k]) / 1e6,
                     100 * act / cu_num / gui,
                     100 * c["SQ_THREAD_CYCLES_VALU"] / (act * 64) if act else 0.0,
                     100 * c["SQ_LDS_BANK_CONFLICT"] / gui / cu_num,
                     c["SQ_LDS_BANK_CONFLICT"],
                     c["SQ_INSTS_VALU"] / c["SQ_WAVES"], c["SQ_INSTS_LDS"] / c["SQ_WAVES"]))
    rows.sort(key=lambda r: -r[1] * r[2])
    out = [f"{'kernel':<66}{'calls':>6}{'avg_ms':>9}{'VALUBusy%':>10}{'VALUUtil%':>10}"
           f"{'LDSBank%':>9}{'bank_cyc':>10}{'VALU/wave':>10}{'LDS/wave':>9}"]
    for k, n, ms, vb, vu, lb, bc, vw, lw in rows:
        out.append(f"{k[:66]:<66}{n:>6}{ms:>9.3f}{vb:>10.1f}{vu:>10.1f}{lb:>9.2f}{bc:>10.3g}"
                   f"{vw:>10.0f}{lw:>9.0f}")
    return "\n".join(out)


def cpu_suite(warmup: int = 2, reps: int = 5, c4_crops: int = 8):
    """The CPU baseline of every configuration: the reference's CPU path (this
    package's PyTorch fallbacks, pinned bit-exact or within tolerance to the
    reference's own fallbacks by the golden vectors) at every configuration,
    forward and backward timed separately with perf_counter (`warmup`
    untimed runs, median of `reps`), on every host core.  c0-c3 run at full
    size; c4 on `c4_crops` 256 x 256 crops per timed run (the rate is per
    pixel-shift, so it extrapolates to the full image).  The oracle's C
    restatement (OpenMP) runs the same inputs as a second, labelled column.
    Yields one dict per (op, config, pass)."""
    import torch

    import oracle
    from neural_shift_cuda import (accumulate_uz, normalized_accumulate_uz, pair_gather,
                                   shift_gather)
    from neural_shift_cuda_amd.workloads import (box_stack, config0_inputs, halfplane_shifts,
                                                 logit_weights, softplus_weights,
                                                 synthetic_image, window_shifts)
    threads = _cpu_threads()
    model = cpu_model()
    oracle.build()

    def med(fn, setup=None):
        ts = []
        for i in range(warmup + reps):
            arg = setup(None) if setup else None
            t0 = time.perf_counter()
            fn(arg)
            dt = time.perf_counter() - t0
            if i >= warmup:
                ts.append(dt)
        return statistics.median(ts)

    def rec(op, cfg, pas, sec, units, oracle_sec=None, note=""):
        d = {"op": op, "config": cfg, "pass": pas, "ms": round(sec * 1e3, 3),
             "mpix_shifts_s": round(units / sec / 1e6, 3) if units else None,
             "threads": threads, "cpu_count": os.cpu_count(), "cpu_model": model,
             "kind": "port", "timing": f"perf_counter, {warmup} warmups, median of {reps}"}
        if oracle_sec is not None:
            d["oracle_c_ms"] = round(oracle_sec * 1e3, 3)
            d["oracle_c_mpix_shifts_s"] = round(units / oracle_sec / 1e6, 3) if units else None
        if note:
            d["note"] = note
        _log(f"cpu {op} {cfg} {pas}: {sec*1e3:.1f} ms")
        return d

    def acc_case(op, cfg, x, w, sh, gU, gZ, normalized=False, log_w=False, crops=None,
                 note=""):
        units = x.numel() * sh.size(0) * (crops or 1)
        f64 = x.dtype == torch.float64
        odt = torch.float64 if f64 else torch.float32

        def fwd(_):
            for _i in range(crops or 1):
                if normalized:
                    normalized_accumulate_uz(x, w, sh, log_weights=log_w, return_log_degree=True,
                                             validate=False)
                else:
                    accumulate_uz(x, w, sh)

        def graph(_):
            xr, wr = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
            if normalized:
                outs = normalized_accumulate_uz(xr, wr, sh, log_weights=log_w,
                                                return_log_degree=True, validate=False)
            else:
                outs = accumulate_uz(xr, wr, sh)
            return outs

        def bwd(outs):
            torch.autograd.backward(list(outs), [gU, gZ])

        tf = med(fwd)
        # backward: the forward graph is built untimed, then one backward
        tb = med(bwd, setup=graph) * (crops or 1)
        if normalized:
            D, L = oracle.normalized(x, w, sh, log_weights=log_w, dtype=odt)
            of = med(lambda _: oracle.normalized(x, w, sh, log_weights=log_w, dtype=odt))
            ob = med(lambda _: oracle.normalized_bwd(x, w, D, L, gU, gZ, sh,
                                                     log_weights=log_w, dtype=odt))
        else:
            of = med(lambda _: oracle.accumulate_uz(x, w, sh, dtype=odt))
            ob = med(lambda _: oracle.accumulate_uz_bwd(x, w, gU, gZ, sh, dtype=odt))
        k = crops or 1
        return [rec(op, cfg, "fwd", tf, units, of * k, note),
                rec(op, cfg, "bwd", tb, units, ob * k, note)]

    out = []
    g = torch.Generator().manual_seed(77)
    # c0: fp32 1x1x256^2, R=3 half-plane, comp_box; forward only (its config)
    x0, w0, sh0 = config0_inputs()
    units0 = x0.numel() * sh0.size(0)
    t = med(lambda _: accumulate_uz(x0, w0, sh0))
    o = med(lambda _: oracle.accumulate_uz(x0, w0, sh0, dtype=torch.float32))
    out.append(rec("accumulate_uz", "c0", "fwd", t, units0, o))
    # c1: gathers, bf16 B=8 C=3 256^2, box (61 rows) and periodic (121 rows)
    for mode, sh in (("box", halfplane_shifts(5)), ("periodic", window_shifts(5))):
        gd = synthetic_image(8, 3, 256, 256, seed=21).to(torch.bfloat16)
        units = gd.numel() * sh.size(0)
        for op, fn, ofn in (("shift_gather", shift_gather, oracle.shift_gather),
                            ("pair_gather", pair_gather, oracle.pair_gather)):
            t = med(lambda _: fn(gd, sh))

            def graph(_, fn=fn):
                gr = gd.clone().requires_grad_(True)
                return gr, fn(gr, sh)[0]

            def bwd(arg):
                gr, out_ = arg
                out_.backward(torch.ones_like(out_))

            tb = med(bwd, setup=graph)
            o = med(lambda _: ofn(gd, sh))
            out.append(rec(op, f"c1 {mode}", "fwd", t, units, o))
            out.append(rec(op, f"c1 {mode}", "bwd", tb, units))
    # c2: fp16 B=4 C=1 512^2 R=7 (S=113): accumulate_uz and normalized (logits)
    sh = halfplane_shifts(7)
    x = synthetic_image(4, 1, 512, 512, seed=205).to(torch.float16)
    w = (softplus_weights((sh.size(0) * 4, 1, 512, 512), seed=206)
         * box_stack(sh, 4, 512, 512)).to(torch.float16)
    gU = torch.randn(4, 1, 512, 512, generator=g)
    gZ = torch.randn(4, 1, 512, 512, generator=g)
    out += acc_case("accumulate_uz", "c2", x, w, sh, gU, gZ)
    lw = logit_weights((sh.size(0) * 4, 1, 512, 512), seed=207).to(torch.float16)
    out += acc_case("normalized_accumulate_uz", "c2 log", x, lw, sh, gU, gZ, normalized=True,
                    log_w=True)
    del x, w, lw
    # c3: GASD full window (121 rows), comp_box; fp32 B=16 and fp64 B=2
    sh = window_shifts(5)
    for dtype, B, tag in ((torch.float32, 16, "c3"), (torch.float64, 2, "c3 fp64")):
        x = synthetic_image(B, 3, 256, 256, seed=301).to(dtype)
        w = (softplus_weights((sh.size(0) * B, 3, 256, 256), seed=302)
             * box_stack(sh, B, 256, 256)).to(dtype)
        acc = torch.float64 if dtype == torch.float64 else torch.float32
        gU = torch.randn(B, 3, 256, 256, generator=g, dtype=acc)
        gZ = torch.randn(B, 3, 256, 256, generator=g, dtype=acc)
        out += acc_case("accumulate_uz", tag, x, w, sh, gU, gZ)
        out += acc_case("normalized_accumulate_uz", tag + " pos", x, w, sh, gU,
                        torch.zeros_like(gZ), normalized=True)
        del x, w
    # c4: 256 x 256 crops of the 8192^2, S=85 workload (the full image would
    # stack about 2 x 169 planes of 268 MB); rate per pixel-shift
    x, w, sh, gU, gZ = _fallback_crop_inputs("c4", 256, 256, 404)
    out += acc_case("accumulate_uz", "c4 crops", x, w, sh, gU, gZ, crops=c4_crops,
                    note=f"{c4_crops} crops of 1x1x256x256 per timed run")
    return out


def suite_cpu(budget_s: float = 1.0):
    """The same (op, config, pass) set as suite(), on the CPU: the oracle's
    reference-order C restatement (OpenMP over all host cores, fp32
    arithmetic for fp16/bf16/fp32 inputs as on the GPU) on a bounded crop of
    each configuration.  Returns {(op, config, pass): (Mpixel-shifts/s,
    sample description)}; the rate is per pixel-shift, so it compares with
    the GPU figure of the full configuration."""
    import torch

    import oracle
    from neural_shift_cuda_amd.workloads import (box_stack, halfplane_shifts, logit_weights,
                                                 synthetic_image, window_shifts)
    oracle.build()

    def rate(fn, units):
        fn()
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            if time.perf_counter() - t0 >= budget_s:
                break
        dt = time.perf_counter() - t0
        return units * reps / dt / 1e6, f"{reps} reps in {dt:.2f}s"

    out = {}
    g = torch.Generator().manual_seed(5)
    f32 = torch.float32
    # c1 gathers (bf16 copies), one image of the batch
    for mode, sh in (("box", halfplane_shifts(5)), ("periodic", window_shifts(5))):
        B, C, H, W = 1, 3, 256, 256
        S, N = sh.size(0), B * C * H * W
        gd = synthetic_image(B, C, H, W, seed=21).to(torch.bfloat16)
        for op, fwd, bwd, k in (("shift_gather", oracle.shift_gather, oracle.shift_gather_bwd, 1),
                                ("pair_gather", oracle.pair_gather, oracle.pair_gather_bwd, 2)):
            go = torch.randn(S * B, k * C, H, W, generator=g).to(torch.bfloat16)
            crop = f"1x{C}x{H}x{W} of c1 (S={S})"
            r, n = rate(lambda: fwd(gd, sh), N * S)
            out[(op, f"c1 {mode}", "fwd")] = (r, f"{crop}, {n}")
            r, n = rate(lambda: bwd(go, sh, B, C, H, W, dtype=f32), N * S)
            out[(op, f"c1 {mode}", "bwd")] = (r, f"{crop}, {n}")

    def acc_pair(op, cfg, x, w, sh, normalized=False, log_w=False):
        B, C, H, W = x.shape
        S, N = sh.size(0), x.numel()
        crop = f"{B}x{C}x{H}x{W} crop of {cfg.split()[0]} (S={S})"
        gU = torch.randn(B, C, H, W, generator=g)
        gZ = torch.randn(B, C, H, W, generator=g)
        if normalized:
            D, L = oracle.normalized(x, w, sh, log_weights=log_w, dtype=f32)
            r, n = rate(lambda: oracle.normalized(x, w, sh, log_weights=log_w, dtype=f32), N * S)
            out[(op, cfg, "fwd")] = (r, f"{crop}, {n}")
            r, n = rate(lambda: oracle.normalized_bwd(x, w, D, L, gU, gZ, sh, log_weights=log_w,
                                                      dtype=f32), N * S)
        else:
            r, n = rate(lambda: oracle.accumulate_uz(x, w, sh, dtype=f32), N * S)
            out[(op, cfg, "fwd")] = (r, f"{crop}, {n}")
            r, n = rate(lambda: oracle.accumulate_uz_bwd(x, w, gU, gZ, sh, dtype=f32), N * S)
        out[(op, cfg, "bwd")] = (r, f"{crop}, {n}")

    def softplus_w(sh, B, C, H, W, box=True):
        w = torch.nn.functional.softplus(torch.randn(sh.size(0) * B, C, H, W, generator=g))
        return w * box_stack(sh, B, H, W) if box else w

    sh = halfplane_shifts(7)
    x = synthetic_image(1, 1, 512, 512, seed=11)
    acc_pair("accumulate_uz", "c2", x, softplus_w(sh, 1, 1, 512, 512), sh)
    lw = logit_weights((sh.size(0), 1, 512, 512), seed=32)
    acc_pair("normalized_accumulate_uz", "c2 log", x, lw, sh, normalized=True, log_w=True)
    sh = window_shifts(5)
    x = synthetic_image(1, 3, 256, 256, seed=11)
    w = softplus_w(sh, 1, 3, 256, 256)
    acc_pair("accumulate_uz", "c3", x, w, sh)
    acc_pair("normalized_accumulate_uz", "c3 pos", x, w, sh, normalized=True)
    x = synthetic_image(1, 1, 1024, 1024, seed=11)
    sh4 = halfplane_shifts(6)
    acc_pair("accumulate_uz", "c4", x, softplus_w(sh4, 1, 1, 1024, 1024), sh4)
    # scalar, c3 shape, one image
    B, C, H, W = 1, 3, 256, 256
    S, N = sh.size(0), B * C * H * W
    x = synthetic_image(B, C, H, W, seed=51)
    ws = torch.rand(S, B, C, generator=g)
    gU = torch.randn(B, C, H, W, generator=g)
    gZ = torch.randn(B, C, H, W, generator=g)
    crop = f"{B}x{C}x{H}x{W} of the c3 shape (S={S})"
    r, n = rate(lambda: oracle.accumulate_uz_scalar(x, ws, sh[:, :2], dtype=f32), N * S)
    out[("accumulate_uz_scalar", "c3 shape", "fwd")] = (r, f"{crop}, {n}")
    r, n = rate(lambda: oracle.accumulate_uz_scalar_bwd(x, ws, gU, gZ, sh[:, :2], dtype=f32),
                N * S)
    out[("accumulate_uz_scalar", "c3 shape", "bwd")] = (r, f"{crop}, {n}")
    # Metropolis c4, a 1024^2 crop
    S4, N = sh4.size(0), 1024 * 1024
    wh = torch.nn.functional.softplus(torch.randn(1, S4, 1, 1024, 1024, generator=g))
    img = synthetic_image(1, 1, 1024, 1024, seed=62)
    r, n = rate(lambda: oracle.metropolis(wh, img, sh4, True, dtype=f32), N * S4)
    out[("metropolis_aggregate", "c4", "fwd")] = (r, f"1x1x1024x1024 crop of c4 (S={S4}), {n}")
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c4", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--suite", action="store_true",
                    help="time every op at its BASELINE config (one JSON line per pass) "
                         "instead of the headline step")
    ap.add_argument("--only", nargs="*", default=None, help="ops for --suite")
    ap.add_argument("--cpu-suite", action="store_true",
                    help="CPU baseline: the PyTorch fallbacks at every config, fwd and "
                         "bwd separately (one JSON line per pass); no GPU")
    ap.add_argument("--cpu-warmup", type=int, default=2, help="untimed runs per pass (--cpu-suite)")
    ap.add_argument("--cpu-reps", type=int, default=5, help="timed runs per pass (--cpu-suite)")
    ap.add_argument("--mall-probe", action="store_true",
                    help="first versus second read of 32 MB-1 GB buffers (Infinity Cache "
                         "reuse) and the streaming probes; one JSON line each")
    ap.add_argument("--summarize-traffic", metavar="PROF_DIR", default=None,
                    help="write profiles/accumulate_uz_bwd_<config>_traffic.json from the "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE runs under PROF_DIR and exit")
    ap.add_argument("--summarize-counters", metavar="RAW_DIR", default=None,
                    help="print per-kernel VALU / LDS metrics from a rocprofv3 --pmc pass of "
                         "bench.COUNTERS written under RAW_DIR and exit")
    a = ap.parse_args()

    if a.summarize_counters:
        print(summarize_counters(a.summarize_counters))
        return 0

    if a.summarize_traffic:
        print(json.dumps(summarize_traffic(a.summarize_traffic, a.config), indent=1))
        return 0

    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; multi-GPU runs are not part "
              "of it (the op shards by batch, or by horizontal bands with R halo rows; "
              "bench.py --suite --only accumulate_uz_band measures one GPU's band)",
              file=sys.stderr)
        return 2

    if a.cpu_suite:
        for d in cpu_suite(a.cpu_warmup, a.cpu_reps):
            print(json.dumps(d), flush=True)
        return 0

    if a.mall_probe:
        import torch
        dev = torch.device("cuda:0")
        print(json.dumps({"stream_probes_gbs": stream_probes(dev)}), flush=True)
        for row in mall_probe(dev):
            print(json.dumps(row), flush=True)
        return 0

    if a.suite:
        import torch
        from neural_shift_cuda_amd import ops
        if not ops._HAS_CUDA_EXT:
            raise RuntimeError(f"HIP library failed to load: {ops._EXT_IMPORT_ERROR}")
        recs = suite(torch.device("cuda:0"), a.steps, a.warmup, a.only)
        if not a.no_cpu_baseline:
            import oracle
            _log("cpu baseline per pass")
            cpu = suite_cpu(a.cpu_budget / 10.0)
            for d in recs:
                key = (d["op"], d["config"], d["pass"])
                if key in cpu:
                    d["cpu_mpix_shifts_s"] = round(cpu[key][0], 2)
                    d["cpu_cores"] = oracle.max_threads()
                    d["cpu_kind"] = "port"
                    d["cpu_sample"] = cpu[key][1]
        for d in recs:
            print(json.dumps(d), flush=True)
        return 0

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
    probes = stream_probes(dev)

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
        # the library's own streaming probes on this box (best of their
        # variants): reference points, not ceilings -- the backward's 1:1
        # read/write stream runs a little above the best probe copy
        "stream_probes_gbs": probes,
        "bwd_vs_probe_copy": round(achieved / probes["copy_gbs"], 4),
        "roofline": {
            "kernel": "accumulate_uz backward pass: accumulate_uz_bwd_scatter_kernel + "
                      "spill_fixup_kernel",
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

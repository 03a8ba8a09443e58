"""Build libneural_shift_hip.so for gfx950 with hipcc (no torch linkage).

    python -m neural_shift_cuda_amd.build [--jobs N]

Every ``csrc/*.hip`` / ``csrc/*.cpp`` file is compiled to an object under
``neural_shift_cuda_amd/_build`` and linked into
``neural_shift_cuda_amd/libneural_shift_hip.so``.  The library exports only
the C ABI declared in ``include/neural_shift_hip.h``.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libneural_shift_hip.so")
INCLUDE = os.path.join(ROOT, "include")
ARCH = "gfx950"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _flags(build_id: str):
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-fvisibility=hidden",
        # Packed FP32 (v_pk_*_f32) generation stays off for all device code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-function",
        "-Wno-unused-command-line-argument",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
        f'-DNSH_BUILD_ID="{build_id}"',
    ]


def _sources():
    return sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC)
        if f.endswith(".hip") or f.endswith(".cpp"))


def _compile(src: str, flags) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [_hipcc(), *flags, *lang, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    noise = "\n".join(
        ln for ln in res.stderr.splitlines()
        if "packed-fp32-ops" not in ln and ln.strip())
    if noise:
        sys.stderr.write(noise + "\n")
    return obj


def build(jobs: int = 0, verbose: bool = True) -> str:
    """Compile and link the library; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    build_id = time.strftime("%Y%m%dT%H%M%S")
    flags = _flags(build_id)
    srcs = _sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    t0 = time.time()
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, flags), srcs))
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           "-Wl,--no-undefined", "-Wl,-z,defs"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[neural_shift_cuda_amd] built {LIB} ({len(srcs)} sources, "
              f"{time.time() - t0:.1f}s)")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=0)
    a = ap.parse_args()
    build(a.jobs)

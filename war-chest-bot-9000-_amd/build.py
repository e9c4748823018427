"""Build libwcwave.so (the wave executor) for gfx950 with hipcc.

Every source is compiled with -ffp-contract=off (no a*b+c contraction: the CFR
state must reproduce the CPU solver's float32 rounding), correctly rounded
float32 division, preserved denormals, and packed-FP32 instructions disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libwcwave.so")
BUILD = os.path.join(HERE, "_build")
ARCH = os.environ.get("WC_OFFLOAD_ARCH", "gfx950")

SOURCES = ["job.cpp", "synth.cpp", "wave.cpp", "capi_host.cpp", "executor.cpp", "service.cpp", "capi_gpu.cpp",
           "kernels.hip", "noalloc.hip", "v5.hip", "probe.hip", "check.hip"]

COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result", "-ffp-contract=off"]
DEVICE = [f"--offload-arch={ARCH}", "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc():
    for c in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON, "-c", os.path.join(SRC, src), "-o", obj]
    if src.endswith(".hip"):
        cmd[1:1] = ["-x", "hip"]
        cmd += DEVICE
    else:
        cmd[1:1] = ["-x", "c++"]
        cmd += ["-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose=False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    jobs = min(len(SOURCES), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    # the throughput tape: a native caller of the C ABI (no HIP code of its own)
    tape = os.path.join(HERE, "wc_tape")
    cmd = [hipcc(), "-x", "c++", *COMMON, os.path.join(SRC, "wave_tape.cpp"), "-o", tape + ".tmp", "-L" + HERE,
           "-lwcwave", "-Wl,-rpath,$ORIGIN", "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"tape build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tape + ".tmp", tape)
    if verbose:
        print(f"built {OUT} and {tape}")
    return OUT


if __name__ == "__main__":
    try:
        build(verbose=True)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)

"""Builds the HIP engine library hk_amd/libhkhip.so (and the benchmark's peak probes,
hk_amd/libhkpeak.so) for gfx950 (hipcc, in-tree).

Every translation unit is compiled with hipcc and linked into one shared library exporting the
C ABI of include/hkhip.h. Flags that matter for the arithmetic:
  -ffp-contract=off   no implicit FMA contraction: the dequantizer is bit-exact with hk's
                      decoders and every fused multiply-add in the kernels is written as fmaf
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      no packed-FP32 instructions
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libhkhip.so")
BUILD_DIR = os.path.join(HERE, "_build")
# mmvq_<format>.hip instantiate the decode kernels per format (the largest part of the build), so
# they compile in parallel; build() always recompiles everything.
MMVQ_FORMATS = ["q4_k", "q6_k", "q5_k", "iq4_xs", "q8_0", "iq4_nl", "q4_0", "q4_1", "q5_0", "q5_1"]
SOURCES = ["engine.hip", "weights.hip", "qact.hip", "mmvq.hip", "mm.hip", "mm2.hip", "mmsk.hip", "mmx.hip", "net.hip"] + \
    [f"mmvq_{f}.hip" for f in MMVQ_FORMATS]
ARCH = "gfx950"


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found: the HIP engine cannot be built")


def cflags() -> list[str]:
    return [
        "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-result", "-Wno-unused-command-line-argument",
    ]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *cflags(), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    noise = "warning: unknown target feature" if "packed-fp32-ops" in r.stderr else None
    for line in r.stderr.splitlines():
        if "error" in line or ("warning" in line and not (noise and noise in line)):
            print(line, file=sys.stderr)
    return obj


def build(jobs: int | None = None) -> str:
    """Compile every source and link libhkhip.so. Always rebuilds."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    build_peak()
    return OUT


PEAK_SRC = "peak.hip"
PEAK_OUT = os.path.join(HERE, "libhkpeak.so")


def build_peak() -> str:
    """The benchmark's peak probes (MFMA rate, HBM read rate): a library of their own."""
    obj = _compile(PEAK_SRC)
    tmp = PEAK_OUT + ".tmp"
    r = subprocess.run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, obj],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, PEAK_OUT)
    return PEAK_OUT


if __name__ == "__main__":
    print(build())

"""Builds liblrs.so (all HIP sources under csrc/) for gfx950 with hipcc, and
the measurement library liblrs_probe.so (probe/probe.hip, used by bench.py
only; not part of the product).

Every HIP translation unit is compiled with
  -ffp-contract=off     the dequant must round like the Rust reference
                        (hot kernels write their FMAs explicitly)
  -packed-fp32-ops off  no v_pk_{add,mul,fma}_f32 is ever emitted
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "liblrs.so")
PROBE_SRC = os.path.join(HERE, "probe", "probe.hip")
PROBE_OUT = os.path.join(HERE, "liblrs_probe.so")
BUILD = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-warning-option",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    # the host pass does not know the packed-fp32 feature; anything else is shown
    for line in r.stderr.splitlines():
        if "packed-fp32-ops" not in line and "warning" in line:
            print(line, file=sys.stderr)
    return obj


def _link(objs, out: str) -> None:
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)


def build(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip"))) + [PROBE_SRC]
    with cf.ThreadPoolExecutor(max_workers=min(jobs, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    _link(objs[:-1], OUT)
    _link(objs[-1:], PROBE_OUT)
    return OUT


if __name__ == "__main__":
    print(build())

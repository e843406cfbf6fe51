"""Build of the measurement library used by bench.py (not part of the product):

  libtbe_floor.so   the gather-floor kernel of measure/gather_floor.hip

It lands next to this file so it travels with the source tree to the GPU box.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
FLOOR_LIB = os.path.join(HERE, "libtbe_floor.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wall", "-Wno-unused-command-line-argument", "-Wno-pass-failed"]


def build() -> None:
    cmd = [os.path.join(ROCM, "bin", "hipcc"), *HIP_FLAGS, "-shared", os.path.join(HERE, "gather_floor.hip"),
           "-o", FLOOR_LIB]
    print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if out.strip():
        print(out, flush=True)
    if r.returncode != 0:
        raise RuntimeError(f"build of {FLOOR_LIB} failed ({r.returncode})")


if __name__ == "__main__":
    build()
    sys.exit(0)

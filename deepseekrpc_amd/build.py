"""Build ``libdsr_sampling.so`` in-tree with hipcc for gfx950.

    python -m deepseekrpc_amd.build

Flags that the numerics depend on:
  -ffp-contract=off   no FMA contraction: the penalty, scaling and ratio
                      arithmetic must round like the reference's NumPy float64
                      (its own CUDA build passes --fmad=false, native/setup.py:19);
  no -ffast-math      IEEE division and float64 denormals are required
                      (temperature 1e-320 is a tested input).
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OUT = os.path.join(HERE, "libdsr_sampling.so")
SOURCES = ["dsr_sampling.hip"]
HEADERS = ["dsr_common.h", "dsr_wave.h", "dsr_general.h", "dsr_fast.h", "dsr_topk.h", "dsr_full.h", "dsr_verify.h", "dsr_history.h", "dsr_split.h", "dsr_numpy.h", "dsr_head.h", "dsr_f32.h"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
    # Packed FP32 instructions stay off (they are not needed on this path).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def build(verbose: bool = False) -> str:
    cmd = [HIPCC, *FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", *[os.path.join(CSRC, s) for s in SOURCES], "-o", OUT + ".tmp"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))

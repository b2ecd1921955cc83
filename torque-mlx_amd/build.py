"""Build recipe for libtorque_hip.so (gfx950).

    python torque-mlx_amd/build.py            # or __graft_entry__.build()

Compiles csrc/torque_hip.hip with hipcc into torque_hip/libtorque_hip.so,
in-tree.  Packed-FP32 VALU ops are disabled for all device code.  The
atomic optimizer is off for device code: it rewrites a single lane's LDS
atomic (the split kernels' tile counter) into a wave-wide form that waits
for the result at once, where the kernels want it one iteration later.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
REPO = ROOT.parent
SOURCE = ROOT / "csrc" / "torque_hip.hip"
OUTPUT = ROOT / "torque_hip" / "libtorque_hip.so"
ARCH = os.environ.get("TORQUE_HIP_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Xarch_device",
    "-mllvm=-amdgpu-atomic-optimizer-strategy=None",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found")
    return path


def build_library(verbose: bool = False) -> Path:
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", str(REPO / "include"), "-I", str(ROOT / "csrc"), str(SOURCE), "-o", str(OUTPUT) + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{stderr}")
    os.replace(str(OUTPUT) + ".tmp", OUTPUT)
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr)
    return OUTPUT


if __name__ == "__main__":
    print(build_library(verbose=True))

"""Build recipe for libtorque_hip.so (gfx950).

    python torque-mlx_amd/build.py            # or __graft_entry__.build()
    python torque-mlx_amd/build.py --asan OUT.so   # host-only AddressSanitizer build

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


# Host-only AddressSanitizer build (argument validation, split planning,
# workspace checks): the host pass is instrumented, the gfx950 code is not.
ASAN_FLAGS = ["-O1", "-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer", "-shared-libasan"]


def asan_runtime() -> Path:
    """The clang AddressSanitizer runtime a process must preload to load the ASan build."""
    hits = sorted(Path(hipcc()).resolve().parents[1].glob("lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not hits:
        raise RuntimeError("libclang_rt.asan-x86_64.so not found next to hipcc")
    return hits[-1]


def build_library(verbose: bool = False, asan: bool = False, output: Path | None = None) -> Path:
    """Compile the library to `output` (default: the in-tree libtorque_hip.so; the ASan build has no
    default location and needs one)."""
    if asan and output is None:
        raise ValueError("the AddressSanitizer build needs an output path outside the package")
    out = Path(output) if output is not None else OUTPUT
    flags = [f for f in HIPCC_FLAGS if not (asan and f == "-O3")] + (ASAN_FLAGS if asan else [])
    cmd = [hipcc(), *flags, "-I", str(REPO / "include"), "-I", str(ROOT / "csrc"), str(SOURCE), "-o", str(out) + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{stderr}")
    os.replace(str(out) + ".tmp", out)
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr)
    return out


if __name__ == "__main__":
    if "--asan" in sys.argv:
        print(build_library(verbose=True, asan=True, output=Path(sys.argv[sys.argv.index("--asan") + 1])))
    else:
        print(build_library(verbose=True))

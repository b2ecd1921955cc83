"""The C-ABI's host code under AddressSanitizer: tests/test_abi.py against a host-instrumented build.

CPU only.  Builds the library with the host pass instrumented (argument
validation, split planning, workspace checks; the gfx950 code is built as
usual) into a temporary directory, then runs test_abi.py in a subprocess that
preloads the clang ASan runtime and loads that build through TORQUE_HIP_LIB.
Leak checking is off: the interpreter's own allocations are not the library's.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]


def test_abi_under_address_sanitizer(tmp_path):
    sys.path.insert(0, str(REPO / "torque-mlx_amd"))
    import build

    lib = build.build_library(asan=True, output=tmp_path / "libtorque_hip_asan.so")
    env = dict(
        os.environ,
        LD_PRELOAD=str(build.asan_runtime()),
        ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
        TORQUE_HIP_LIB=str(lib),
    )
    r = subprocess.run(
        [sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", str(REPO / "tests" / "test_abi.py")],
        env=env, capture_output=True, text=True, timeout=900, cwd=REPO,
    )
    assert "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert " passed" in r.stdout

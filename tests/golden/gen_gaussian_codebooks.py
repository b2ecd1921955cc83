"""Write golden vectors for the Gaussian Lloyd-Max codebook builder.

``build_gaussian_codebook`` (reference ``src/torque_mlx/quantization.py:89-117``)
depends on numpy's PCG64 normal stream, ``np.quantile`` and an early-stopped
Lloyd iteration, so no closed form pins its exact float32 output.  This script
loads the reference's own ``quantization.py`` by file path (it imports only the
standard library and numpy) and records its output for the parameter sets the
reference's defaults and tests use.  It runs only in the build container, where
the reference is mounted; the JSON it writes is what the tests read.

    python tests/golden/gen_gaussian_codebooks.py /root/reference
"""

from __future__ import annotations

import importlib.util
import json
import sys
from pathlib import Path

import numpy as np

CASES = [
    # (bit_width, seed, sample_size, iterations)
    *[(b, s, 200_000, 32) for b in (2, 3, 4) for s in (0, 1, 2, 3, 7, 8)],
    (4, 7, 20_000, 12),  # test_quantization.py:114-121
    (4, 2, 50_000, 16),  # test_error_budget.py:7-17
]


def main() -> None:
    reference_root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    module_path = reference_root / "src" / "torque_mlx" / "quantization.py"
    spec = importlib.util.spec_from_file_location("_reference_quantization", module_path)
    module = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = module  # dataclasses resolve annotations through sys.modules
    spec.loader.exec_module(module)

    records = []
    for bit_width, seed, sample_size, iterations in CASES:
        codebook = module.build_gaussian_codebook(
            bit_width, seed=seed, sample_size=sample_size, iterations=iterations
        )
        boundaries = module.codebook_boundaries(codebook)
        records.append(
            {
                "bit_width": bit_width,
                "seed": seed,
                "sample_size": sample_size,
                "iterations": iterations,
                "centroids_hex": [f"{v:08x}" for v in np.asarray(codebook.centroids, np.float32).view(np.uint32)],
                "boundaries_hex": [f"{v:08x}" for v in np.asarray(boundaries, np.float32).view(np.uint32)],
                "centroids": [float(v) for v in codebook.centroids],
                "name": codebook.name,
            }
        )
    out = Path(__file__).with_name("gaussian_codebooks.json")
    out.write_text(
        json.dumps({"numpy_version": np.__version__, "source": "quantization.py:89-136", "cases": records}, indent=1),
        encoding="utf-8",
    )
    print(f"wrote {len(records)} codebooks to {out}")


if __name__ == "__main__":
    main()

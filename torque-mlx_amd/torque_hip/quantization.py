"""Codebooks and packed geometry (reference quantization.py).

Codebook construction is one-time host setup, as in the reference.  The
per-token quantize / pack / unpack work runs on the GPU: see
``torque_hip.ops.quantize_and_pack_rows`` and the cache classes.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from math import ceil
from pathlib import Path

import numpy as np

SUPPORTED_BIT_WIDTHS = {2, 3, 4}
WORD_BITS = 32


def _validate_bit_width(bit_width: int) -> None:
    if bit_width not in SUPPORTED_BIT_WIDTHS:
        raise ValueError(f"Unsupported bit width: {bit_width}")


@dataclass(frozen=True)
class Codebook:
    """Sorted float32 scalar codebook with 2^b centroids (quantization.py:21-65)."""

    bit_width: int
    centroids: np.ndarray
    name: str = "gaussian_lloyd_max"

    def __post_init__(self) -> None:
        _validate_bit_width(self.bit_width)
        object.__setattr__(self, "centroids", np.asarray(self.centroids, dtype=np.float32))
        expected = 1 << self.bit_width
        if self.centroids.ndim != 1 or self.centroids.size != expected:
            raise ValueError(
                f"Expected {expected} centroids for {self.bit_width}-bit codebook, got shape {self.centroids.shape}",
            )
        if not np.all(np.diff(self.centroids) >= 0):
            raise ValueError("Centroids must be sorted in ascending order")

    def to_dict(self) -> dict[str, object]:
        return {"bit_width": self.bit_width, "centroids": self.centroids.tolist(), "name": self.name}

    def to_json(self) -> str:
        return json.dumps(self.to_dict(), indent=2, sort_keys=True)

    @classmethod
    def from_dict(cls, payload: dict[str, object]) -> "Codebook":
        return cls(
            bit_width=int(payload["bit_width"]),
            centroids=np.asarray(payload["centroids"], dtype=np.float32),
            name=str(payload.get("name", "gaussian_lloyd_max")),
        )

    @classmethod
    def from_json(cls, payload: str) -> "Codebook":
        return cls.from_dict(json.loads(payload))


def save_codebook(codebook: Codebook, path: str | Path) -> None:
    Path(path).write_text(codebook.to_json(), encoding="utf-8")


def load_codebook(path: str | Path) -> Codebook:
    return Codebook.from_json(Path(path).read_text(encoding="utf-8"))


def packed_words_for_head_dim(head_dim: int, bit_width: int) -> int:
    """uint32 words per packed vector, ceil(D * b / 32) (quantization.py:76-81)."""
    _validate_bit_width(bit_width)
    if head_dim <= 0:
        raise ValueError("head_dim must be positive")
    return ceil((head_dim * bit_width) / WORD_BITS)


def kv_bytes_per_token(head_dim: int, bit_width: int, kv_heads: int = 1) -> int:
    """Packed K+V bytes per token (quantization.py:84-86)."""
    return packed_words_for_head_dim(head_dim=head_dim, bit_width=bit_width) * 4 * kv_heads * 2


def build_gaussian_codebook(
    bit_width: int,
    *,
    iterations: int = 32,
    sample_size: int = 200_000,
    seed: int = 0,
) -> Codebook:
    """Lloyd-Max codebook for N(0, 1) (quantization.py:89-117).

    Quantile initialisation over ``sample_size`` seeded normal samples, then
    up to ``iterations`` Lloyd steps (nearest-boundary assignment, cluster
    means in float64), stopping when the centroids no longer move.
    """
    _validate_bit_width(bit_width)
    rng = np.random.default_rng(seed)
    samples = rng.normal(loc=0.0, scale=1.0, size=sample_size).astype(np.float32)
    levels = 1 << bit_width
    centroids = np.quantile(samples, np.linspace(0.0, 1.0, levels + 2, dtype=np.float32)[1:-1]).astype(np.float32)
    for _ in range(iterations):
        edges = (centroids[:-1] + centroids[1:]) / 2.0
        members = np.searchsorted(edges, samples, side="right")
        updated = centroids.copy()
        for level in range(levels):
            cluster = samples[members == level]
            if cluster.size:
                updated[level] = cluster.mean(dtype=np.float64)
        converged = np.allclose(updated, centroids)
        centroids = updated
        if converged:
            break
    return Codebook(bit_width=bit_width, centroids=np.sort(centroids))


def build_uniform_codebook(bit_width: int) -> Codebook:
    """linspace(-1, 1, 2^b) codebook used by the reference benchmarks (benchmarking.py:16-21)."""
    return Codebook(
        bit_width=bit_width,
        centroids=np.linspace(-1.0, 1.0, 1 << bit_width, dtype=np.float32),
        name="uniform",
    )


def codebook_boundaries(codebook: "Codebook | np.ndarray") -> np.ndarray:
    """float32 decision boundaries (c_i + c_{i+1}) / 2 (quantization.py:128-136)."""
    centroids = (
        np.asarray(codebook.centroids, dtype=np.float32)
        if isinstance(codebook, Codebook)
        else np.asarray(codebook, dtype=np.float32)
    )
    if centroids.ndim != 1 or centroids.size < 2:
        raise ValueError("Expected at least two sorted centroids to build quantization boundaries")
    return ((centroids[:-1] + centroids[1:]) / 2.0).astype(np.float32)

"""Structured Hadamard rotation Pi = D1 H D2 / sqrt(D) (reference rotation.py).

Sign vectors are drawn on the host exactly as the reference does; applying the
rotation runs the wavefront FWHT kernel (``tq_fwht``), whose float32 output is
bit-identical to the reference's numpy transform.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum
from typing import Any

import numpy as np
import torch

from torque_hip import _lib
from torque_hip._tensors import device, dtype_code, shape_of, stream_handle, to_device


class RotationMode(str, Enum):
    HADAMARD = "hadamard"

    def __str__(self) -> str:
        return self.value


def validate_head_dim(head_dim: int) -> None:
    if head_dim not in {64, 128, 256}:
        raise ValueError(f"Unsupported head dimension for rotation: {head_dim}")


def _rotate(values: Any, signs_left: torch.Tensor, signs_right: torch.Tensor, *, inverse: bool) -> torch.Tensor:
    dev = signs_left.device
    x = to_device(values, dev)
    head_dim = int(x.shape[-1]) if x.dim() else 0
    validate_head_dim(head_dim)
    y = torch.empty(x.shape, dtype=torch.float32, device=dev)
    rows = x.numel() // head_dim
    _lib.call(
        "tq_fwht",
        x.data_ptr(),
        dtype_code(x),
        y.data_ptr(),
        rows,
        head_dim,
        signs_left.data_ptr(),
        signs_right.data_ptr(),
        1 if inverse else 0,
        stream_handle(dev),
    )
    return y


@dataclass(frozen=True)
class RotationSpec:
    """Pi = D1 H D2 with D1 = diag(signs_left), D2 = diag(signs_right) (rotation.py:51-106)."""

    head_dim: int
    signs_left: np.ndarray
    signs_right: np.ndarray
    seed: int | None = None

    def __post_init__(self) -> None:
        validate_head_dim(self.head_dim)
        object.__setattr__(self, "signs_left", np.asarray(self.signs_left, dtype=np.float32))
        object.__setattr__(self, "signs_right", np.asarray(self.signs_right, dtype=np.float32))
        if self.signs_left.shape != (self.head_dim,) or self.signs_right.shape != (self.head_dim,):
            raise ValueError("Rotation sign vectors must match head_dim")
        object.__setattr__(self, "_device_signs", {})

    @classmethod
    def from_seed(cls, head_dim: int, seed: int = 0) -> "RotationSpec":
        """Signs drawn from ``numpy.random.default_rng(seed)``, left first (rotation.py:75-86)."""
        validate_head_dim(head_dim)
        rng = np.random.default_rng(seed)
        signs_left = rng.choice(np.array([-1.0, 1.0], dtype=np.float32), size=head_dim)
        signs_right = rng.choice(np.array([-1.0, 1.0], dtype=np.float32), size=head_dim)
        return cls(head_dim=head_dim, signs_left=signs_left, signs_right=signs_right, seed=seed)

    def device_signs(self, dev: torch.device | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        dev = dev or device()
        cache = self._device_signs  # type: ignore[attr-defined]
        key = str(dev)
        if key not in cache:
            cache[key] = (
                torch.from_numpy(self.signs_left.copy()).to(dev),
                torch.from_numpy(self.signs_right.copy()).to(dev),
            )
        return cache[key]

    def _check(self, values: Any) -> None:
        shape = shape_of(values)
        if not shape or shape[-1] != self.head_dim:
            raise ValueError(f"Expected last dimension {self.head_dim}, got {shape[-1] if shape else shape}")

    def apply_device(self, values: Any) -> torch.Tensor:
        """Pi x on the GPU; returns a float32 device tensor."""
        self._check(values)
        left, right = self.device_signs(values.device if isinstance(values, torch.Tensor) and values.is_cuda else None)
        return _rotate(values, left, right, inverse=False)

    def inverse_device(self, values: Any) -> torch.Tensor:
        """Pi^-1 y on the GPU; returns a float32 device tensor."""
        self._check(values)
        left, right = self.device_signs(values.device if isinstance(values, torch.Tensor) and values.is_cuda else None)
        return _rotate(values, left, right, inverse=True)

    def apply(self, values: Any) -> Any:
        """Pi x.  numpy in -> numpy out; torch in -> float32 device tensor out."""
        out = self.apply_device(values)
        return out if isinstance(values, torch.Tensor) else out.cpu().numpy()

    def inverse(self, values: Any) -> Any:
        out = self.inverse_device(values)
        return out if isinstance(values, torch.Tensor) else out.cpu().numpy()

    def matrix(self) -> np.ndarray:
        """Pi as a dense matrix, apply(I).T (rotation.py:104-106)."""
        return self.apply(np.eye(self.head_dim, dtype=np.float32)).T


def apply_structured_rotation(values: Any, head_dim: int, seed: int = 0) -> Any:
    return RotationSpec.from_seed(head_dim=head_dim, seed=seed).apply(values)


def apply_structured_rotation_hip(values: Any, *, signs_left: Any, signs_right: Any) -> torch.Tensor:
    """Device rotation with explicit signs (replaces apply_structured_rotation_mlx, rotation.py:113-123)."""
    head_dim = shape_of(values)[-1]
    spec = RotationSpec(head_dim=head_dim, signs_left=_host(signs_left), signs_right=_host(signs_right))
    return spec.apply_device(values)


def inverse_structured_rotation_hip(values: Any, *, signs_left: Any, signs_right: Any) -> torch.Tensor:
    """Device inverse rotation with explicit signs (replaces inverse_structured_rotation_mlx, rotation.py:126-136)."""
    head_dim = shape_of(values)[-1]
    spec = RotationSpec(head_dim=head_dim, signs_left=_host(signs_left), signs_right=_host(signs_right))
    return spec.inverse_device(values)


def _host(values: Any) -> np.ndarray:
    if isinstance(values, torch.Tensor):
        return values.detach().cpu().numpy().astype(np.float32)
    return np.asarray(values, dtype=np.float32)


# Reference names of the device rotation helpers.
apply_structured_rotation_mlx = apply_structured_rotation_hip
inverse_structured_rotation_mlx = inverse_structured_rotation_hip

"""Runtime configuration (reference config.py:8-42)."""

from __future__ import annotations

from dataclasses import dataclass

from torque_hip.layout import PackedKVLayout, build_variant_id
from torque_hip.quantization import SUPPORTED_BIT_WIDTHS
from torque_hip.rotation import RotationMode, validate_head_dim

SUPPORTED_SCALE_MODES: tuple[str, ...] = ("none", "rms")


@dataclass(frozen=True)
class TorqueConfig:
    """Top-level runtime configuration; same fields, defaults and errors as the reference.

    ``scale_mode`` is an opt-in extension (the reference has no per-vector
    scales; its codes index one global codebook per stream,
    quantization.py:120-148): "none" (default) stores exactly the reference's
    codes; "rms" quantizes every rotated key/value vector divided by its RMS
    and keeps that RMS as one float32 per (layer, KV head, token) and stream.
    """

    bit_width: int = 4
    head_dim: int = 128
    num_layers: int = 1
    kv_heads: int = 1
    fused_weights: bool = False
    rotation_mode: RotationMode = RotationMode.HADAMARD
    rotation_seed: int = 0
    scale_mode: str = "none"

    def validate(self) -> None:
        if self.bit_width not in SUPPORTED_BIT_WIDTHS:
            raise ValueError(f"Unsupported bit width: {self.bit_width}")
        validate_head_dim(self.head_dim)
        if self.num_layers <= 0:
            raise ValueError("num_layers must be positive")
        if self.kv_heads <= 0:
            raise ValueError("kv_heads must be positive")
        if self.scale_mode not in SUPPORTED_SCALE_MODES:
            raise ValueError("scale_mode must be one of " + ", ".join(SUPPORTED_SCALE_MODES))

    @property
    def layout(self) -> PackedKVLayout:
        self.validate()
        return PackedKVLayout(bit_width=self.bit_width, head_dim=self.head_dim)

    @property
    def variant_id(self) -> str:
        self.validate()
        variant = build_variant_id(
            bit_width=self.bit_width,
            head_dim=self.head_dim,
            fused_weights=self.fused_weights,
            rotation_mode=RotationMode(self.rotation_mode).value,
        )
        return variant if self.scale_mode == "none" else f"{variant}-{self.scale_mode}"

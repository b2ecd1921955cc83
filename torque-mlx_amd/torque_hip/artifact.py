"""Converted-model artifact and its ``build_cache()`` (reference artifact.py:17-347).

An artifact is ``manifest.json`` plus ``weights.npz`` (fused W_Q, W_K, W_V,
W_O).  ``build_cache()`` returns the HIP-backed ``TorqueKVCache`` configured
with the artifact's runtime config and codebooks.  Weight fusion and
conversion are offline tooling and are not part of this package; loading
reads the manifest as JSON and the weights with ``numpy.load`` (no pickle).
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Mapping

import numpy as np

from torque_hip.cache import TorqueKVCache
from torque_hip.config import TorqueConfig
from torque_hip.quantization import Codebook
from torque_hip.rotation import RotationMode

ARTIFACT_FORMAT = "torque-mlx-artifact"
ARTIFACT_VERSION = 1
DEFAULT_WEIGHTS_FILE = "weights.npz"
DEFAULT_MANIFEST_FILE = "manifest.json"


def _json_ready(value: Any) -> Any:
    if isinstance(value, dict):
        return {str(k): _json_ready(v) for k, v in value.items()}
    if isinstance(value, (list, tuple)):
        return [_json_ready(v) for v in value]
    if isinstance(value, np.generic):
        return value.item()
    return value


def _require_fields(payload: Mapping[str, object], names: tuple[str, ...]) -> None:
    missing = [name for name in names if name not in payload]
    if missing:
        raise ValueError(f"Missing required fields: {', '.join(missing)}")


def config_from_dict(payload: Mapping[str, object]) -> TorqueConfig:
    return TorqueConfig(
        bit_width=int(payload["bit_width"]),
        head_dim=int(payload["head_dim"]),
        num_layers=int(payload["num_layers"]),
        kv_heads=int(payload["kv_heads"]),
        fused_weights=bool(payload["fused_weights"]),
        rotation_mode=RotationMode(str(payload["rotation_mode"])),
        rotation_seed=int(payload["rotation_seed"]),
        scale_mode=str(payload.get("scale_mode", "none")),
    )


def config_to_dict(config: TorqueConfig) -> dict[str, object]:
    """The reference's runtime_config fields; ``scale_mode`` (an extension) only when it is not "none", so
    manifests of the reference format stay byte-identical."""
    out: dict[str, object] = {
        "bit_width": config.bit_width,
        "head_dim": config.head_dim,
        "num_layers": config.num_layers,
        "kv_heads": config.kv_heads,
        "fused_weights": config.fused_weights,
        "rotation_mode": RotationMode(config.rotation_mode).value,
        "rotation_seed": config.rotation_seed,
    }
    if config.scale_mode != "none":
        out["scale_mode"] = config.scale_mode
    return out


@dataclass(frozen=True)
class FusedAttentionWeights:
    w_q: np.ndarray
    w_k: np.ndarray
    w_v: np.ndarray
    w_o: np.ndarray
    rotation_seed: int


@dataclass(frozen=True)
class TorqueArtifactManifest:
    """Manifest fields and validation of artifact.py:39-137."""

    model_name: str
    architecture: str
    source_format: str
    runtime_config: TorqueConfig
    key_codebook: Codebook
    value_codebook: Codebook
    weights_file: str = DEFAULT_WEIGHTS_FILE
    format_name: str = ARTIFACT_FORMAT
    format_version: int = ARTIFACT_VERSION
    weight_names: dict[str, str] = field(default_factory=lambda: {"w_q": "w_q", "w_k": "w_k", "w_v": "w_v", "w_o": "w_o"})
    extra_metadata: dict[str, object] = field(default_factory=dict)

    def __post_init__(self) -> None:
        self.runtime_config.validate()
        if not self.runtime_config.fused_weights:
            raise ValueError("Artifact runtime_config must enable fused_weights")
        if self.format_name != ARTIFACT_FORMAT:
            raise ValueError(f"Unsupported artifact format: {self.format_name}")
        if self.format_version != ARTIFACT_VERSION:
            raise ValueError(f"Unsupported artifact version: {self.format_version}")

    @classmethod
    def from_dict(cls, payload: Mapping[str, object]) -> "TorqueArtifactManifest":
        _require_fields(
            payload, ("model_name", "architecture", "source_format", "runtime_config", "key_codebook", "value_codebook")
        )
        runtime_payload = payload["runtime_config"]
        if not isinstance(runtime_payload, Mapping):
            raise ValueError("runtime_config must be an object")
        weight_names = dict(payload.get("weight_names", {})) or {"w_q": "w_q", "w_k": "w_k", "w_v": "w_v", "w_o": "w_o"}
        return cls(
            model_name=str(payload["model_name"]),
            architecture=str(payload["architecture"]),
            source_format=str(payload["source_format"]),
            runtime_config=config_from_dict(runtime_payload),
            key_codebook=Codebook.from_dict(dict(payload["key_codebook"])),
            value_codebook=Codebook.from_dict(dict(payload["value_codebook"])),
            weights_file=str(payload.get("weights_file", DEFAULT_WEIGHTS_FILE)),
            format_name=str(payload.get("format_name", ARTIFACT_FORMAT)),
            format_version=int(payload.get("format_version", ARTIFACT_VERSION)),
            weight_names={str(k): str(v) for k, v in weight_names.items()},
            extra_metadata={str(k): _json_ready(v) for k, v in dict(payload.get("extra_metadata", {})).items()},
        )

    def to_dict(self) -> dict[str, object]:
        return {
            "format_name": self.format_name,
            "format_version": self.format_version,
            "model_name": self.model_name,
            "architecture": self.architecture,
            "source_format": self.source_format,
            "variant_id": self.runtime_config.variant_id,
            "runtime_config": config_to_dict(self.runtime_config),
            "weights_file": self.weights_file,
            "weight_names": dict(self.weight_names),
            "key_codebook": self.key_codebook.to_dict(),
            "value_codebook": self.value_codebook.to_dict(),
            "extra_metadata": _json_ready(self.extra_metadata),
        }


@dataclass(frozen=True)
class TorqueArtifact:
    manifest: TorqueArtifactManifest
    fused_weights: FusedAttentionWeights | None = None

    @property
    def runtime_config(self) -> TorqueConfig:
        return self.manifest.runtime_config

    @property
    def key_codebook(self) -> Codebook:
        return self.manifest.key_codebook

    @property
    def value_codebook(self) -> Codebook:
        return self.manifest.value_codebook

    def build_cache(self) -> TorqueKVCache:
        """HIP-backed cache with the artifact's config and codebooks (artifact.py:157-162)."""
        return TorqueKVCache(
            config=self.runtime_config,
            key_codebook=self.key_codebook,
            value_codebook=self.value_codebook,
        )

    @classmethod
    def load(cls, directory: str | Path) -> "TorqueArtifact":
        """Read manifest.json and weights.npz (artifact.py:224-243)."""
        target = Path(directory)
        manifest_path = target / DEFAULT_MANIFEST_FILE
        if not manifest_path.exists():
            raise FileNotFoundError(f"Artifact manifest not found: {manifest_path}")
        manifest = TorqueArtifactManifest.from_dict(json.loads(manifest_path.read_text(encoding="utf-8")))
        weights_path = target / manifest.weights_file
        if not weights_path.exists():
            raise FileNotFoundError(f"Artifact weights not found: {weights_path}")
        with np.load(weights_path, allow_pickle=False) as data:
            names = manifest.weight_names
            weights = FusedAttentionWeights(
                w_q=np.asarray(data[names["w_q"]], dtype=np.float32),
                w_k=np.asarray(data[names["w_k"]], dtype=np.float32),
                w_v=np.asarray(data[names["w_v"]], dtype=np.float32),
                w_o=np.asarray(data[names["w_o"]], dtype=np.float32),
                rotation_seed=manifest.runtime_config.rotation_seed,
            )
        return cls(manifest=manifest, fused_weights=weights)


def load_torque_artifact(directory: str | Path) -> TorqueArtifact:
    return TorqueArtifact.load(directory)

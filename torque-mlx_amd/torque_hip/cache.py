"""``TorqueKVCache`` -- the reference's runtime cache API (cache.py:35-227),
backed by device slabs and the HIP append / decode kernels.

Same constructor, methods, shape forms, squeeze rules and ``ValueError``
messages as the reference.  One extension (reference cache_mlx.py:724-740):
``decode`` also accepts grouped-query queries [L, Hq, D] with Hq a multiple of
kv_heads; query head q reads KV head q // (Hq / kv_heads).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch

from torque_hip._slab import SlabStore
from torque_hip._tensors import codes_to_numpy, device, shape_of, to_device
from torque_hip.config import TorqueConfig
from torque_hip.layout import CacheMetadata
from torque_hip.quantization import Codebook, build_gaussian_codebook
from torque_hip.rotation import RotationMode, RotationSpec

DEFAULT_INITIAL_CAPACITY = 256


@dataclass
class TorqueKVCache:
    """Rotation-native packed KV cache (one token per ``append``)."""

    config: TorqueConfig = field(default_factory=TorqueConfig)
    key_codebook: Codebook | None = None
    value_codebook: Codebook | None = None
    sequence_length: int = 0
    rotation: RotationSpec = field(init=False, repr=False)
    _store: SlabStore = field(init=False, repr=False)

    def __post_init__(self) -> None:
        self.config.validate()
        self.key_codebook = self.key_codebook or build_gaussian_codebook(
            self.config.bit_width, seed=self.config.rotation_seed
        )
        self.value_codebook = self.value_codebook or build_gaussian_codebook(
            self.config.bit_width, seed=self.config.rotation_seed + 1
        )
        self.rotation = RotationSpec.from_seed(head_dim=self.config.head_dim, seed=self.config.rotation_seed)
        self._store = SlabStore(
            self.config,
            self.key_codebook,
            self.value_codebook,
            self.rotation,
            initial_capacity=DEFAULT_INITIAL_CAPACITY,
            growth_factor=2,
            dev=device(),
        )
        self.sequence_length = 0

    @property
    def metadata(self) -> CacheMetadata:
        return CacheMetadata(
            variant_id=self.config.variant_id,
            bit_width=self.config.bit_width,
            head_dim=self.config.head_dim,
            num_layers=self.config.num_layers,
            kv_heads=self.config.kv_heads,
            rotation_mode=RotationMode(self.config.rotation_mode).value,
            fused_weights=self.config.fused_weights,
            codebook_name=self.key_codebook.name,
        )

    @property
    def _key_codes(self) -> torch.Tensor:
        """Packed key slab [L, Hkv, capacity, W] (uint32 view)."""
        return self._store.key_codes.view(torch.uint32)

    @property
    def _value_codes(self) -> torch.Tensor:
        return self._store.value_codes.view(torch.uint32)

    def append(self, *, key: Any, value: Any) -> None:
        """Append one decode step for all layers and KV heads (cache.py:78-96)."""
        keys = self._normalize_layer_heads(key, "key")
        values = self._normalize_layer_heads(value, "value")
        self._store.append(keys.unsqueeze(2), values.unsqueeze(2), rotate_keys=True, rotate_values=True)
        self.sequence_length += 1

    def append_many(self, *, key: Any, value: Any) -> None:
        """Bulk append of S tokens, keys/values [L, Hkv, S, D]; same codes as S single appends."""
        cfg = self.config
        shape = shape_of(key)
        if len(shape) != 4 or shape[:2] != (cfg.num_layers, cfg.kv_heads) or shape[3] != cfg.head_dim:
            raise ValueError(f"key must have shape ({cfg.num_layers}, {cfg.kv_heads}, seq_len, {cfg.head_dim}), got {shape}")
        if shape_of(value) != shape:
            raise ValueError(f"key/value sequence dimensions must match, got {shape} and {shape_of(value)}")
        keys = to_device(key, self._store.device)
        values = to_device(value, self._store.device)
        self._store.append(keys, values, rotate_keys=True, rotate_values=True)
        self.sequence_length += shape[2]

    def decode(self, *, query: Any) -> np.ndarray:
        """Packed decode attention for one query step (cache.py:98-140)."""
        out = self.decode_device(query=query)
        return self._squeeze(out.cpu().numpy())

    def decode_mlx(self, *, query: Any) -> np.ndarray:
        """The reference's device-decode entry (cache.py:142-180); same HIP path as ``decode``."""
        return self.decode(query=query)

    def decode_device(self, *, query: Any) -> torch.Tensor:
        """Decode returning the unsqueezed [L, Hq, D] float32 device tensor."""
        queries = self._normalize_queries(query)
        if self.sequence_length == 0:
            return torch.zeros(queries.shape, dtype=torch.float32, device=queries.device)
        return self._store.decode(queries, rotate_query=True, inverse_output=not self.config.fused_weights)

    def reset(self) -> None:
        self.sequence_length = 0
        self._store.reset()

    def export_dequantized(self) -> tuple[np.ndarray, np.ndarray]:
        """Dequantized rotated cache contents [L, Hkv, S, D] (cache.py:189-214)."""
        keys, values = self._store.export_dequantized()
        return keys.cpu().numpy(), values.cpu().numpy()

    def packed_codes(self) -> tuple[np.ndarray, np.ndarray]:
        """Packed words of the stored tokens, uint32 [L, Hkv, S, W]."""
        s = self.sequence_length
        return (
            codes_to_numpy(self._store.key_codes[:, :, :s]),
            codes_to_numpy(self._store.value_codes[:, :, :s]),
        )

    # -------------------------------------------------------------- shapes

    def _normalize_layer_heads(self, values: Any, label: str) -> torch.Tensor:
        """[D] (1 layer / 1 head), [Hkv, D] (1 layer) or [L, Hkv, D] (cache.py:216-227)."""
        shape = shape_of(values)
        cfg = self.config
        target = (cfg.num_layers, cfg.kv_heads, cfg.head_dim)
        if shape == (cfg.head_dim,):
            if target[:2] != (1, 1):
                raise ValueError(f"{label} shape {shape} only valid for 1 layer / 1 head")
        elif not (shape == (cfg.kv_heads, cfg.head_dim) and cfg.num_layers == 1) and shape != target:
            raise ValueError(f"{label} must have shape {target}, got {shape}")
        return to_device(values, self._store.device).reshape(target)

    def _normalize_queries(self, values: Any) -> torch.Tensor:
        shape = shape_of(values)
        cfg = self.config
        target = (cfg.num_layers, cfg.kv_heads, cfg.head_dim)
        if shape == (cfg.head_dim,):
            if target[:2] != (1, 1):
                raise ValueError(f"query shape {shape} only valid for 1 layer / 1 head")
            heads = 1
        elif len(shape) == 2 and cfg.num_layers == 1 and shape[1] == cfg.head_dim and shape[0] % cfg.kv_heads == 0:
            heads = shape[0]
        elif len(shape) == 3 and shape[0] == cfg.num_layers and shape[2] == cfg.head_dim and shape[1] % cfg.kv_heads == 0:
            heads = shape[1]
        else:
            raise ValueError(f"query must have shape {target}, got {shape}")
        return to_device(values, self._store.device).reshape(cfg.num_layers, heads, cfg.head_dim)

    def _squeeze(self, outputs: np.ndarray) -> np.ndarray:
        if self.config.num_layers == 1 and outputs.shape[1] == 1:
            return outputs[0, 0]
        if self.config.num_layers == 1:
            return outputs[0]
        return outputs

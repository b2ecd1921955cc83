"""``TorqueKVCacheHIP`` -- drop-in for the reference's device cache
``TorqueKVCacheMLX`` (cache_mlx.py:40-799), on MI355X.

Same constructor knobs, methods, shape forms, strategies, flags and errors.
Storage is the reference slab layout [L, Hkv, capacity, W] in HBM.  Every
append packs immediately (one fused rotate -> quantize -> pack launch for all
layers, heads and tokens); ``decode_tail_capacity`` is accepted, validated and
reported through ``capacity`` but no dense fp16 tail is kept, so decode reads
exactly the packed cache the numpy reference would hold.  Decode is one launch
of the split-K packed attention kernel for all layers and query heads.

Strategies: "split_batched" (default) and "auto" use the split-K kernel with
the default split count; "fused_per_head" uses the same kernel with one split
per head group.  With ``profile_decode_components`` the decode is run as the
reference's three stages (score kernel, softmax kernel, value kernel), each
timed with HIP events into ``last_decode_profile``; ``decode_with_current``
and ``decode_append`` then run the reference's staged path with the current
token (its score and value share timed as ``tail_seconds``; decode_append as
that decode followed by the append, ``append_seconds``).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from math import sqrt
from typing import Any, Literal

import numpy as np
import torch

from torque_hip import ops
from torque_hip._slab import EventTimer, SlabStore
from torque_hip._tensors import device, shape_of, to_device
from torque_hip.config import TorqueConfig
from torque_hip.layout import CacheMetadata
from torque_hip.quantization import Codebook, build_gaussian_codebook
from torque_hip.rotation import RotationMode, RotationSpec

DecodeStrategy = Literal["auto", "split_batched", "fused_per_head"]
SUPPORTED_DECODE_STRATEGIES: tuple[str, ...] = ("auto", "split_batched", "fused_per_head")


@dataclass
class TorqueKVCacheHIP:
    config: TorqueConfig = field(default_factory=TorqueConfig)
    key_codebook: Codebook | None = None
    value_codebook: Codebook | None = None
    initial_capacity: int = 256
    growth_factor: int = 2
    decode_tail_capacity: int = 16
    decode_strategy: str = "split_batched"
    profile_decode_components: bool = False
    rotate_keys_on_append: bool = True
    rotate_values_on_append: bool = True
    rotate_queries_on_decode: bool = True
    sequence_length: int = 0
    rotation: RotationSpec = field(init=False, repr=False)
    last_decode_profile: dict[str, float] = field(init=False, repr=False)
    _store: SlabStore = field(init=False, repr=False)

    def __post_init__(self) -> None:
        self.config.validate()
        if self.initial_capacity <= 0:
            raise ValueError("initial_capacity must be positive")
        if self.growth_factor < 2:
            raise ValueError("growth_factor must be at least 2")
        if self.decode_tail_capacity < 0:
            raise ValueError("decode_tail_capacity must be non-negative")
        if self.decode_strategy not in SUPPORTED_DECODE_STRATEGIES:
            raise ValueError("decode_strategy must be one of " + ", ".join(SUPPORTED_DECODE_STRATEGIES))
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
            initial_capacity=self.initial_capacity,
            growth_factor=self.growth_factor,
            dev=device(),
        )
        self.sequence_length = 0
        self.last_decode_profile = {}

    # -------------------------------------------------------------- properties

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
    def capacity(self) -> int:
        return self._store.capacity + self.decode_tail_capacity

    @property
    def offset(self) -> int:
        return self.sequence_length

    @property
    def state(self) -> tuple[torch.Tensor, torch.Tensor]:
        return self._key_codes, self._value_codes

    @property
    def _key_codes(self) -> torch.Tensor:
        return self._store.key_codes.view(torch.uint32)

    @property
    def _value_codes(self) -> torch.Tensor:
        return self._store.value_codes.view(torch.uint32)

    # -------------------------------------------------------------- append

    def append(self, *, key: Any, value: Any) -> None:
        self.append_many(key=key, value=value)

    def append_many(self, *, key: Any, value: Any) -> None:
        """Append S >= 1 tokens for all layers and KV heads (cache_mlx.py:151-171)."""
        keys = self._normalize_layer_heads_sequence(key, "key")
        values = self._normalize_layer_heads_sequence(value, "value")
        if tuple(keys.shape[:3]) != tuple(values.shape[:3]):
            raise ValueError(
                f"key/value sequence dimensions must match, got {tuple(keys.shape)} and {tuple(values.shape)}",
            )
        profile = self.last_decode_profile if self.profile_decode_components else None
        with EventTimer(profile, "append_seconds", self._store.device):
            self._store.append(
                keys,
                values,
                rotate_keys=self.rotate_keys_on_append,
                rotate_values=self.rotate_values_on_append,
            )
        self.sequence_length += int(keys.shape[2])

    append_many_mlx = append_many

    # -------------------------------------------------------------- decode

    def decode(self, *, query: Any, return_numpy: bool = True) -> Any:
        """Decode one query step for all layers and query heads (cache_mlx.py:173-234)."""
        self.last_decode_profile = {}
        queries = self._normalize_query_heads(query, "query")
        query_heads = int(queries.shape[1])
        if self.sequence_length == 0:
            zeros = torch.zeros((self.config.num_layers, query_heads, self.config.head_dim), device=queries.device)
            return self._finalize_output(zeros, query_heads=query_heads, return_numpy=return_numpy)
        self._check_groups(query_heads)
        outputs = self._decode_packed(queries)
        return self._finalize_output(outputs, query_heads=query_heads, return_numpy=return_numpy)

    decode_mlx = decode

    def decode_with_current(self, *, query: Any, key: Any, value: Any, return_numpy: bool = True) -> Any:
        """Decode over the cache plus the current (not yet appended) token (cache_mlx.py:236-302)."""
        self.last_decode_profile = {}
        queries = self._normalize_query_heads(query, "query")
        current_keys = self._normalize_layer_heads_sequence(key, "key")
        current_values = self._normalize_layer_heads_sequence(value, "value")
        if int(current_keys.shape[2]) != 1 or int(current_values.shape[2]) != 1:
            raise ValueError("decode_mlx_with_current expects a single current token for key/value")
        query_heads = int(queries.shape[1])
        self._check_groups(query_heads)
        current = self._store.quantize_current(
            current_keys,
            current_values,
            rotate_keys=self.rotate_keys_on_append,
            rotate_values=self.rotate_values_on_append,
        )
        profile = self.last_decode_profile if self.profile_decode_components else None
        if self._staged_profile(profile):
            outputs = self._decode_with_current_staged(queries, current, profile)
        else:
            with EventTimer(profile, "packed_decode_seconds", self._store.device):
                outputs = self._store.decode(
                    queries,
                    rotate_query=self.rotate_queries_on_decode,
                    inverse_output=not self.config.fused_weights,
                    current=current,
                    n_splits=self._n_splits(),
                )
        return self._finalize_output(outputs, query_heads=query_heads, return_numpy=return_numpy)

    decode_mlx_with_current = decode_with_current

    def decode_append(self, *, query: Any, key: Any, value: Any, return_numpy: bool = True) -> Any:
        """``decode_with_current`` followed by ``append`` of the same token, in one kernel launch.

        The reference's Qwen decode step makes exactly this pair of calls per layer
        (qwen_mlx.py:826-828).  The packed words written are identical to ``append``'s and the output
        matches ``decode_with_current``'s to float rounding; the cache grows by one token.
        """
        self.last_decode_profile = {}
        queries = self._normalize_query_heads(query, "query")
        keys = self._normalize_layer_heads_sequence(key, "key")
        values = self._normalize_layer_heads_sequence(value, "value")
        if int(keys.shape[2]) != 1 or int(values.shape[2]) != 1:
            raise ValueError("decode_append expects a single token for key/value")
        query_heads = int(queries.shape[1])
        self._check_groups(query_heads)
        profile = self.last_decode_profile if self.profile_decode_components else None
        if self._staged_profile(profile):
            # profiling: the two calls this launch replaces, the decode staged as the reference times it
            current = self._store.quantize_current(
                keys, values, rotate_keys=self.rotate_keys_on_append, rotate_values=self.rotate_values_on_append
            )
            outputs = self._decode_with_current_staged(queries, current, profile)
            with EventTimer(profile, "append_seconds", self._store.device):
                self._store.append(
                    keys, values, rotate_keys=self.rotate_keys_on_append, rotate_values=self.rotate_values_on_append
                )
        else:
            with EventTimer(profile, "packed_decode_seconds", self._store.device):
                outputs = self._store.decode_append(
                    queries,
                    keys,
                    values,
                    rotate_query=self.rotate_queries_on_decode,
                    inverse_output=not self.config.fused_weights,
                    rotate_keys=self.rotate_keys_on_append,
                    rotate_values=self.rotate_values_on_append,
                    n_splits=self._n_splits(),
                )
        self.sequence_length += 1
        return self._finalize_output(outputs, query_heads=query_heads, return_numpy=return_numpy)

    def resolve_decode_strategy(self, *, sequence_length: int | None = None) -> str:
        if self.decode_strategy != "auto":
            return self.decode_strategy
        return "split_batched"

    def reset(self) -> None:
        self.sequence_length = 0
        self._store.reset()

    def make_mask(self, N: int, *, window_size: int | None = None, return_array: bool = False) -> Any:
        """Attention mask for N new tokens at the current offset (cache_mlx.py:322-338)."""
        if N == 1:
            return None
        if not return_array and (window_size is None or N <= window_size):
            return "causal"
        offset = self.offset
        rinds = torch.arange(offset + N)
        linds = torch.arange(offset, offset + N) if offset else rinds
        linds = linds[:, None]
        rinds = rinds[None]
        mask = linds >= rinds
        if window_size is not None:
            mask = mask & (linds < rinds + window_size)
        return mask

    def export_dequantized(self) -> tuple[np.ndarray, np.ndarray]:
        keys, values = self._store.export_dequantized()
        return keys.cpu().numpy(), values.cpu().numpy()

    # -------------------------------------------------------------- internals

    def _n_splits(self) -> int | None:
        return 1 if self.resolve_decode_strategy() == "fused_per_head" else None

    def _check_groups(self, query_heads: int) -> None:
        if query_heads % self.config.kv_heads != 0:
            raise ValueError(
                f"query head count {query_heads} must be divisible by kv_heads {self.config.kv_heads}",
            )

    def _staged_profile(self, profile: dict[str, float] | None) -> bool:
        """Profiling runs the reference's staged split path; it has no per-vector scales, so scaled
        caches time the fused decode instead."""
        return profile is not None and self.resolve_decode_strategy() == "split_batched" and not self._store.scaled

    def _decode_packed(self, queries: torch.Tensor) -> torch.Tensor:
        profile = self.last_decode_profile if self.profile_decode_components else None
        if self._staged_profile(profile):
            return self._decode_staged(queries, profile)
        with EventTimer(profile, "packed_decode_seconds", self._store.device):
            return self._store.decode(
                queries,
                rotate_query=self.rotate_queries_on_decode,
                inverse_output=not self.config.fused_weights,
                n_splits=self._n_splits(),
            )

    def _decode_staged(self, queries: torch.Tensor, profile: dict[str, float]) -> torch.Tensor:
        """The reference's three-stage split path (cache_mlx.py:752-775), each stage timed."""
        cfg, store = self.config, self._store
        dev = store.device
        num_layers, query_heads = int(queries.shape[0]), int(queries.shape[1])
        group = query_heads // cfg.kv_heads
        with EventTimer(profile, "query_rotation_seconds", dev):
            q_rot = self.rotation.apply_device(queries) if self.rotate_queries_on_decode else queries.float()
        s = store.length
        layer_idx = torch.arange(num_layers, device=dev).repeat_interleave(query_heads)
        kv_idx = (torch.arange(query_heads, device=dev) // group).repeat(num_layers)
        k_rows = store.key_codes[layer_idx, kv_idx, :s]
        v_rows = store.value_codes[layer_idx, kv_idx, :s]
        q_flat = q_rot.reshape(num_layers * query_heads, cfg.head_dim).contiguous()
        with EventTimer(profile, "packed_score_seconds", dev):
            scores = ops.score_packed_query_batched(
                q_flat, k_rows, store.key_centroids, bit_width=cfg.bit_width, head_dim=cfg.head_dim
            )
        with EventTimer(profile, "softmax_seconds", dev):
            weights = ops.softmax_rows(scores, 1.0 / sqrt(cfg.head_dim))
        with EventTimer(profile, "packed_value_seconds", dev):
            out_rot = ops.accumulate_packed_values_batched(
                weights, v_rows, store.value_centroids, bit_width=cfg.bit_width, head_dim=cfg.head_dim
            )
        if cfg.fused_weights:
            out = out_rot
        else:
            with EventTimer(profile, "inverse_rotation_seconds", dev):
                out = self.rotation.inverse_device(out_rot)
        return out.reshape(num_layers, query_heads, cfg.head_dim)

    def _decode_with_current_staged(
        self, queries: torch.Tensor, current: tuple[torch.Tensor, torch.Tensor], profile: dict[str, float]
    ) -> torch.Tensor:
        """The reference's staged decode with one current token (cache_mlx.py:565-640), each stage timed:
        the current token's score (tail_seconds), the packed scores, one softmax over the packed scores
        and the current score, the packed value sum, the current value's share (tail_seconds)."""
        cfg, store = self.config, self._store
        dev = store.device
        num_layers, query_heads = int(queries.shape[0]), int(queries.shape[1])
        group = query_heads // cfg.kv_heads
        with EventTimer(profile, "query_rotation_seconds", dev):
            q_rot = self.rotation.apply_device(queries) if self.rotate_queries_on_decode else queries.float()
        layer_idx = torch.arange(num_layers, device=dev).repeat_interleave(query_heads)
        kv_idx = (torch.arange(query_heads, device=dev) // group).repeat(num_layers)
        q_flat = q_rot.reshape(num_layers * query_heads, cfg.head_dim).contiguous()
        cur_k, cur_v = current[0][layer_idx, kv_idx], current[1][layer_idx, kv_idx]  # [B, D], rotated, dequantized
        with EventTimer(profile, "tail_seconds", dev):
            current_scores = (cur_k * q_flat).sum(dim=1, keepdim=True)
        s = store.length
        if s == 0:
            with EventTimer(profile, "tail_seconds", dev):
                out_rot = cur_v.clone()
        else:
            k_rows = store.key_codes[layer_idx, kv_idx, :s]
            v_rows = store.value_codes[layer_idx, kv_idx, :s]
            with EventTimer(profile, "packed_score_seconds", dev):
                scores = ops.score_packed_query_batched(
                    q_flat, k_rows, store.key_centroids, bit_width=cfg.bit_width, head_dim=cfg.head_dim
                )
            with EventTimer(profile, "softmax_seconds", dev):
                weights = ops.softmax_rows(torch.cat([scores, current_scores], dim=1), 1.0 / sqrt(cfg.head_dim))
            with EventTimer(profile, "packed_value_seconds", dev):
                packed_out = ops.accumulate_packed_values_batched(
                    weights[:, :s].contiguous(), v_rows, store.value_centroids, bit_width=cfg.bit_width,
                    head_dim=cfg.head_dim,
                )
            with EventTimer(profile, "tail_seconds", dev):
                out_rot = packed_out + cur_v * weights[:, s:]
        if cfg.fused_weights:
            out = out_rot
        else:
            with EventTimer(profile, "inverse_rotation_seconds", dev):
                out = self.rotation.inverse_device(out_rot)
        return out.reshape(num_layers, query_heads, cfg.head_dim)

    def _finalize_output(self, outputs: torch.Tensor, *, query_heads: int, return_numpy: bool) -> Any:
        if not return_numpy:
            return outputs
        output_np = outputs.cpu().numpy()
        if self.config.num_layers == 1 and query_heads == 1:
            return output_np[0, 0]
        if self.config.num_layers == 1:
            return output_np[0]
        return output_np

    def _normalize_layer_heads_sequence(self, values: Any, label: str) -> torch.Tensor:
        """Accepted forms (cache_mlx.py:442-466): [D], [Hkv, D], [L, Hkv, D], [Hkv, S, D], [L, Hkv, S, D]."""
        cfg = self.config
        shape = shape_of(values)
        target = (cfg.num_layers, cfg.kv_heads, cfg.head_dim)
        dev = self._store.device
        if len(shape) == 1 and shape == (cfg.head_dim,):
            if target[:2] != (1, 1):
                raise ValueError(f"{label} shape {shape} only valid for 1 layer / 1 head")
            return to_device(values, dev).reshape(1, 1, 1, cfg.head_dim)
        if len(shape) == 2 and shape == (cfg.kv_heads, cfg.head_dim):
            if cfg.num_layers != 1:
                raise ValueError(f"{label} shape {shape} only valid for 1 layer")
            return to_device(values, dev).reshape(1, cfg.kv_heads, 1, cfg.head_dim)
        if len(shape) == 3:
            if shape == target:
                return to_device(values, dev).reshape(cfg.num_layers, cfg.kv_heads, 1, cfg.head_dim)
            if cfg.num_layers == 1 and shape[0] == cfg.kv_heads and shape[2] == cfg.head_dim:
                return to_device(values, dev).reshape(1, cfg.kv_heads, shape[1], cfg.head_dim)
        if len(shape) == 4 and shape[0] == cfg.num_layers and shape[1] == cfg.kv_heads and shape[3] == cfg.head_dim:
            return to_device(values, dev)
        raise ValueError(
            f"{label} must have shape ({cfg.num_layers}, {cfg.kv_heads}, seq_len, {cfg.head_dim}) "
            f"or a compatible single-token form, got {shape}",
        )

    def _normalize_query_heads(self, values: Any, label: str) -> torch.Tensor:
        """Accepted forms (cache_mlx.py:724-740): [D], [Hq, D] (1 layer), [L, Hq, D]."""
        cfg = self.config
        shape = shape_of(values)
        dev = self._store.device
        if len(shape) == 1 and shape == (cfg.head_dim,):
            if (cfg.num_layers, cfg.kv_heads) != (1, 1):
                raise ValueError(f"{label} shape {shape} only valid for 1 layer / 1 head")
            return to_device(values, dev).reshape(1, 1, cfg.head_dim)
        if len(shape) == 2 and shape[1] == cfg.head_dim and cfg.num_layers == 1:
            return to_device(values, dev).reshape(1, shape[0], cfg.head_dim)
        if len(shape) == 3 and shape[0] == cfg.num_layers and shape[2] == cfg.head_dim:
            return to_device(values, dev)
        raise ValueError(
            f"{label} must have shape ({cfg.num_layers}, query_heads, {cfg.head_dim}) "
            f"or a compatible 1-layer form, got {shape}",
        )


# Reference class name: code written against the MLX cache runs unchanged.
TorqueKVCacheMLX = TorqueKVCacheHIP

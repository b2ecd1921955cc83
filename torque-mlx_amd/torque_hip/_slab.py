"""Device slab store shared by the cache classes.

Packed codes live in two int32 tensors (the uint32 bit patterns) of shape
[L, Hkv, capacity, W] -- the reference's canonical layout
(docs/contracts/packed-kv-layout.md:5-10, cache_mlx.py:105-109).  Capacity
grows geometrically like cache_mlx.py:353-371.  With ``scale_mode="rms"`` two
float32 scale slabs [L, Hkv, capacity] sit beside them (one per-vector scale
per token and stream) and every kernel call takes its ``_scaled`` form.
"""

from __future__ import annotations

from time import perf_counter

import torch

from torque_hip import _lib
from torque_hip._tensors import dtype_code, stream_handle
from torque_hip.config import TorqueConfig
from torque_hip.ops import packed_decode, packed_decode_append
from torque_hip.quantization import Codebook, codebook_boundaries
from torque_hip.rotation import RotationSpec


def _kv_pair(keys: torch.Tensor, values: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """K/V in one dtype without rounding either: kept when they already agree, else both float32.

    The reference quantizes float32 K/V (cache_mlx.py:442-466); float16 inputs
    convert to float32 exactly in the kernels, so only a mixed pair needs a
    cast, and it must go up, never down to the narrower type.
    """
    if keys.dtype != values.dtype:
        keys, values = keys.to(torch.float32), values.to(torch.float32)
    return keys.contiguous(), values.contiguous()


class SlabStore:
    def __init__(
        self,
        config: TorqueConfig,
        key_codebook: Codebook,
        value_codebook: Codebook,
        rotation: RotationSpec,
        *,
        initial_capacity: int,
        growth_factor: int,
        dev: torch.device,
    ) -> None:
        self.config = config
        self.layout = config.layout
        self.device = dev
        self.growth_factor = growth_factor
        self.capacity = initial_capacity
        shape = (config.num_layers, config.kv_heads, initial_capacity, self.layout.packed_words)
        self.key_codes = torch.zeros(shape, dtype=torch.int32, device=dev)
        self.value_codes = torch.zeros_like(self.key_codes)
        self.scaled = config.scale_mode == "rms"
        self.key_scales = torch.zeros(shape[:3], dtype=torch.float32, device=dev) if self.scaled else None
        self.value_scales = torch.zeros(shape[:3], dtype=torch.float32, device=dev) if self.scaled else None
        self.key_centroids = torch.from_numpy(key_codebook.centroids.copy()).to(dev)
        self.value_centroids = torch.from_numpy(value_codebook.centroids.copy()).to(dev)
        self.key_boundaries = torch.from_numpy(codebook_boundaries(key_codebook)).to(dev)
        self.value_boundaries = torch.from_numpy(codebook_boundaries(value_codebook)).to(dev)
        self.signs_left, self.signs_right = rotation.device_signs(dev)
        self.length = 0

    # -------------------------------------------------------------- storage

    def ensure_capacity(self, min_capacity: int) -> None:
        if min_capacity <= self.capacity:
            return
        new_capacity = self.capacity
        while new_capacity < min_capacity:
            new_capacity *= self.growth_factor
        shape = (self.config.num_layers, self.config.kv_heads, new_capacity, self.layout.packed_words)
        new_k = torch.zeros(shape, dtype=torch.int32, device=self.device)
        new_v = torch.zeros_like(new_k)
        new_k[:, :, : self.length].copy_(self.key_codes[:, :, : self.length])
        new_v[:, :, : self.length].copy_(self.value_codes[:, :, : self.length])
        self.key_codes, self.value_codes = new_k, new_v
        if self.scaled:
            new_ks = torch.zeros(shape[:3], dtype=torch.float32, device=self.device)
            new_vs = torch.zeros_like(new_ks)
            new_ks[:, :, : self.length].copy_(self.key_scales[:, :, : self.length])
            new_vs[:, :, : self.length].copy_(self.value_scales[:, :, : self.length])
            self.key_scales, self.value_scales = new_ks, new_vs
        self.capacity = new_capacity

    def reset(self) -> None:
        self.length = 0
        self.key_codes.zero_()
        self.value_codes.zero_()
        if self.scaled:
            self.key_scales.zero_()
            self.value_scales.zero_()

    # -------------------------------------------------------------- kernels

    def append(self, keys: torch.Tensor, values: torch.Tensor, *, rotate_keys: bool, rotate_values: bool) -> None:
        """keys/values [L, Hkv, S_new, D] (float32 or float16, same dtype) -> packed in place."""
        seq_new = int(keys.shape[2])
        if seq_new == 0:
            return
        keys, values = _kv_pair(keys, values)
        self.ensure_capacity(self.length + seq_new)
        flags = (_lib.TQ_ROTATE_KEYS if rotate_keys else 0) | (_lib.TQ_ROTATE_VALUES if rotate_values else 0)
        cfg = self.config
        scale_args = (self.key_scales.data_ptr(), self.value_scales.data_ptr()) if self.scaled else ()
        _lib.call(
            "tq_append_scaled" if self.scaled else "tq_append",
            keys.data_ptr(),
            values.data_ptr(),
            dtype_code(keys),
            cfg.num_layers,
            cfg.kv_heads,
            seq_new,
            cfg.head_dim,
            cfg.bit_width,
            self.signs_left.data_ptr(),
            self.signs_right.data_ptr(),
            flags,
            self.key_boundaries.data_ptr(),
            self.value_boundaries.data_ptr(),
            self.key_codes.data_ptr(),
            self.value_codes.data_ptr(),
            *scale_args,
            self.capacity,
            self.length,
            stream_handle(self.device),
        )
        self.length += seq_new

    def quantize_current(
        self, keys: torch.Tensor, values: torch.Tensor, *, rotate_keys: bool, rotate_values: bool
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Rotate -> quantize -> dequantize one token per (layer, KV head): [L, Hkv, 1, D] -> [L, Hkv, D]."""
        cfg = self.config
        keys, values = _kv_pair(keys, values)
        rows = cfg.num_layers * cfg.kv_heads
        k_out = torch.empty((cfg.num_layers, cfg.kv_heads, cfg.head_dim), dtype=torch.float32, device=self.device)
        v_out = torch.empty_like(k_out)
        flags = (_lib.TQ_ROTATE_KEYS if rotate_keys else 0) | (_lib.TQ_ROTATE_VALUES if rotate_values else 0)
        _lib.call(
            "tq_quantize_dequantize_scaled" if self.scaled else "tq_quantize_dequantize",
            keys.data_ptr(),
            values.data_ptr(),
            dtype_code(keys),
            rows,
            cfg.head_dim,
            cfg.bit_width,
            self.signs_left.data_ptr(),
            self.signs_right.data_ptr(),
            flags,
            self.key_boundaries.data_ptr(),
            self.value_boundaries.data_ptr(),
            self.key_centroids.data_ptr(),
            self.value_centroids.data_ptr(),
            k_out.data_ptr(),
            v_out.data_ptr(),
            stream_handle(self.device),
        )
        return k_out, v_out

    def decode(
        self,
        queries: torch.Tensor,
        *,
        rotate_query: bool,
        inverse_output: bool,
        current: tuple[torch.Tensor, torch.Tensor] | None = None,
        n_splits: int | None = None,
    ) -> torch.Tensor:
        """queries [L, Hq, D] -> out [L, Hq, D] float32 on the device."""
        cfg = self.config
        return packed_decode(
            queries,
            num_layers=cfg.num_layers,
            query_heads=int(queries.shape[1]),
            kv_heads=cfg.kv_heads,
            head_dim=cfg.head_dim,
            bit_width=cfg.bit_width,
            key_codes=self.key_codes,
            value_codes=self.value_codes,
            capacity=self.capacity,
            seq_len=self.length,
            key_centroids=self.key_centroids,
            value_centroids=self.value_centroids,
            signs_left=self.signs_left,
            signs_right=self.signs_right,
            rotate_query=rotate_query,
            inverse_output=inverse_output,
            current_keys=None if current is None else current[0],
            current_values=None if current is None else current[1],
            n_splits=n_splits,
            key_scales=self.key_scales,
            value_scales=self.value_scales,
        )

    def decode_append(
        self,
        queries: torch.Tensor,
        keys: torch.Tensor,
        values: torch.Tensor,
        *,
        rotate_query: bool,
        inverse_output: bool,
        rotate_keys: bool,
        rotate_values: bool,
        n_splits: int | None = None,
    ) -> torch.Tensor:
        """Append one token (keys/values [L, Hkv, 1, D]) and decode with it: one launch.

        Scaled slabs take three launches (dequantize the token, decode with it,
        append it): the fused launch packs codes but writes no scales.
        """
        if self.scaled:
            current = self.quantize_current(keys, values, rotate_keys=rotate_keys, rotate_values=rotate_values)
            out = self.decode(queries, rotate_query=rotate_query, inverse_output=inverse_output, current=current,
                              n_splits=n_splits)
            self.append(keys, values, rotate_keys=rotate_keys, rotate_values=rotate_values)
            return out
        cfg = self.config
        self.ensure_capacity(self.length + 1)
        keys, values = _kv_pair(keys, values)
        out = packed_decode_append(
            queries,
            keys,
            values,
            num_layers=cfg.num_layers,
            query_heads=int(queries.shape[1]),
            kv_heads=cfg.kv_heads,
            head_dim=cfg.head_dim,
            bit_width=cfg.bit_width,
            key_codes=self.key_codes,
            value_codes=self.value_codes,
            capacity=self.capacity,
            seq_len=self.length,
            key_centroids=self.key_centroids,
            value_centroids=self.value_centroids,
            key_boundaries=self.key_boundaries,
            value_boundaries=self.value_boundaries,
            signs_left=self.signs_left,
            signs_right=self.signs_right,
            rotate_keys=rotate_keys,
            rotate_values=rotate_values,
            rotate_query=rotate_query,
            inverse_output=inverse_output,
            n_splits=n_splits,
        )
        self.length += 1
        return out

    def export_dequantized(self) -> tuple[torch.Tensor, torch.Tensor]:
        """Dequantized rotated contents [L, Hkv, S, D] (float32, device)."""
        cfg = self.config
        groups = cfg.num_layers * cfg.kv_heads
        shape = (cfg.num_layers, cfg.kv_heads, self.length, cfg.head_dim)
        keys = torch.zeros(shape, dtype=torch.float32, device=self.device)
        values = torch.zeros_like(keys)
        for codes, cent, scales, out in (
            (self.key_codes, self.key_centroids, self.key_scales, keys),
            (self.value_codes, self.value_centroids, self.value_scales, values),
        ):
            scale_args = (scales.data_ptr(),) if self.scaled else ()
            _lib.call(
                "tq_unpack_dequantize_scaled" if self.scaled else "tq_unpack_dequantize",
                codes.data_ptr(),
                *scale_args,
                groups,
                self.capacity,
                self.length,
                cfg.head_dim,
                cfg.bit_width,
                cent.data_ptr(),
                out.data_ptr(),
                stream_handle(self.device),
            )
        return keys, values


class EventTimer:
    """Accumulates GPU time of a region into a profile dict (seconds)."""

    def __init__(self, profile: dict[str, float] | None, key: str, dev: torch.device) -> None:
        self.profile, self.key, self.dev = profile, key, dev

    def __enter__(self) -> "EventTimer":
        if self.profile is not None:
            self.start = torch.cuda.Event(enable_timing=True)
            self.stop = torch.cuda.Event(enable_timing=True)
            self.start.record()
            self.t0 = perf_counter()
        return self

    def __exit__(self, *exc) -> None:
        if self.profile is None:
            return
        self.stop.record()
        self.stop.synchronize()
        self.profile[self.key] = self.profile.get(self.key, 0.0) + self.start.elapsed_time(self.stop) / 1000.0

"""Synthetic decode benchmark (reference benchmarking.py:16-86) on the HIP path.

Same inputs, call sequence and result keys as ``run_synthetic_decode_benchmark``:
seeded N(0, 1) keys / values / query, a ``TorqueKVCache`` with the default
Gaussian codebooks, ``seq_len`` appended tokens, one timed decode, a one-token
decode (TTFT proxy) and the unquantized float32 rotated-attention baseline.
Here the baseline runs on the GPU too (rotation kernel + dense fp32 decode
kernel), and the result adds device-side figures: decode kernel time, packed
KV bytes and achieved HBM bandwidth.
"""

from __future__ import annotations

from time import perf_counter

import numpy as np
import torch

from torque_hip import _lib, ops
from torque_hip._tensors import device
from torque_hip.cache import TorqueKVCache
from torque_hip.config import TorqueConfig
from torque_hip.quantization import build_uniform_codebook, kv_bytes_per_token

HBM_PEAK_GBPS = 8000.0

__all__ = ["build_uniform_codebook", "run_synthetic_decode_benchmark", "HBM_PEAK_GBPS"]


def _timed(fn) -> tuple[object, float]:
    torch.cuda.synchronize()
    started = perf_counter()
    out = fn()
    torch.cuda.synchronize()
    return out, perf_counter() - started


def run_synthetic_decode_benchmark(
    *,
    seq_len: int,
    head_dim: int,
    kv_heads: int,
    bit_width: int,
    seed: int,
    rotation_seed: int | None = None,
) -> dict[str, float]:
    dev = device()
    rng = np.random.default_rng(seed)
    config = TorqueConfig(
        bit_width=bit_width,
        head_dim=head_dim,
        num_layers=1,
        kv_heads=kv_heads,
        rotation_seed=seed if rotation_seed is None else rotation_seed,
    )
    cache = TorqueKVCache(config=config)
    keys = rng.normal(size=(seq_len, kv_heads, head_dim)).astype(np.float32)
    values = rng.normal(size=(seq_len, kv_heads, head_dim)).astype(np.float32)
    query = rng.normal(size=(kv_heads, head_dim)).astype(np.float32)

    k_dev = torch.from_numpy(np.ascontiguousarray(keys.transpose(1, 0, 2))).to(dev)  # [Hkv, S, D]
    v_dev = torch.from_numpy(np.ascontiguousarray(values.transpose(1, 0, 2))).to(dev)
    cache.append_many(key=k_dev[None], value=v_dev[None])

    first_token_cache = TorqueKVCache(config=config, key_codebook=cache.key_codebook, value_codebook=cache.value_codebook)
    first_token_cache.append(key=keys[0], value=values[0])

    cache.decode(query=query)  # warm the kernels once
    quantized_out, quantized_elapsed = _timed(lambda: cache.decode(query=query))
    _, first_decode_elapsed = _timed(lambda: first_token_cache.decode(query=query))

    # Unquantized baseline: rotate K, V, q (bit-identical FWHT kernel), dense fp32 decode, inverse rotation.
    rotation = cache.rotation
    q_dev = torch.from_numpy(query).to(dev)[None]

    def baseline():
        kr = rotation.apply_device(k_dev)[None]
        vr = rotation.apply_device(v_dev)[None]
        sl, sr = rotation.device_signs(dev)
        return ops.dense_decode(
            q_dev, kr, vr, num_layers=1, query_heads=kv_heads, kv_heads=kv_heads, head_dim=head_dim,
            capacity=seq_len, seq_len=seq_len, signs_left=sl, signs_right=sr, rotate_query=True,
            inverse_output=True,
        )

    baseline()
    baseline_out, baseline_elapsed = _timed(baseline)
    baseline_np = baseline_out[0].cpu().numpy()

    # Kernel-only timing of the packed decode (events bound to the launch).
    queries = cache._normalize_queries(query)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 20
    start.record()
    for _ in range(reps):
        cache._store.decode(queries, rotate_query=True, inverse_output=True)
    stop.record()
    stop.synchronize()
    kernel_s = start.elapsed_time(stop) / 1000.0 / reps
    packed_bytes = kv_bytes_per_token(head_dim, bit_width, kv_heads) * seq_len

    max_abs_error = float(np.max(np.abs(quantized_out - baseline_np)))
    return {
        "seq_len": float(seq_len),
        "head_dim": float(head_dim),
        "kv_heads": float(kv_heads),
        "bit_width": float(bit_width),
        "naive_quantized_decode_ms": quantized_elapsed * 1_000.0,
        "naive_quantized_tokens_per_sec": 1.0 / quantized_elapsed,
        "ttft_proxy_ms": first_decode_elapsed * 1_000.0,
        "reference_decode_ms": baseline_elapsed * 1_000.0,
        "reference_tokens_per_sec": 1.0 / baseline_elapsed,
        "kv_bytes_per_token": float(kv_bytes_per_token(head_dim, bit_width, kv_heads)),
        "max_abs_error_vs_rotated_reference": max_abs_error,
        "backend": "hip",
        "decode_kernel_us": kernel_s * 1e6,
        "packed_kv_bytes": float(packed_bytes),
        "hbm_gbps": packed_bytes / kernel_s / 1e9,
        "pct_peak": 100.0 * packed_bytes / kernel_s / 1e9 / HBM_PEAK_GBPS,
        "library": str(_lib.library_path().name),
    }

"""qwen-decode benchmark (reference qwen_benchmark.py:27-493) on the HIP path.

Loads the decode geometry of a local Qwen snapshot (``config.json``) or a
converted torque snapshot (``torque_qwen_manifest.json``), then runs the
KV-growing decode loop: prefill ``prefill_tokens`` tokens, then per step append
one token per layer and decode one query step for all layers and query heads.
Inputs are ``uniform(-1, 1)`` as in the reference (qwen_benchmark.py:274-297)
and the torque cache uses uniform codebooks (:356-357).

Comparators: the reference times MLX-LM's fp16 ``KVCache`` + SDPA and its
``QuantizedKVCache``.  Here the fp16 comparator is the fp16-dense HIP decode
kernel over an fp16 slab updated in place (reported under the reference's
``mlx_fp16_*`` keys and the explicit ``fp16_dense_*`` keys); MLX-LM's
quantized cache has no counterpart and its fields are reported as zero.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from time import perf_counter
from typing import Any, Callable, Mapping

import numpy as np
import torch

from torque_hip import ops
from torque_hip._tensors import device
from torque_hip.artifact import config_from_dict
from torque_hip.cache_hip import SUPPORTED_DECODE_STRATEGIES, TorqueKVCacheHIP
from torque_hip.config import TorqueConfig
from torque_hip.quantization import Codebook, build_uniform_codebook, kv_bytes_per_token

QWEN_MODEL_MANIFEST_FILE = "torque_qwen_manifest.json"
SUPPORTED_QWEN_MODEL_TYPES = {"qwen3_5", "qwen3_5_text"}
DEFAULT_QWEN_DECODE_TAIL_CAPACITY = 8
DEFAULT_QWEN_LARGE_MODEL_DECODE_TAIL_CAPACITY = 0
QWEN_SMALL_MODEL_HIDDEN_SIZE_THRESHOLD = 2048


def resolve_qwen_decode_tail_capacity(*, hidden_size: int | None, requested: int | None) -> int:
    """Tail heuristic of qwen_mlx.py:18-30: 8 below hidden size 2048, else 0."""
    if requested is not None:
        return requested
    if hidden_size is None or hidden_size < QWEN_SMALL_MODEL_HIDDEN_SIZE_THRESHOLD:
        return DEFAULT_QWEN_DECODE_TAIL_CAPACITY
    return DEFAULT_QWEN_LARGE_MODEL_DECODE_TAIL_CAPACITY


@dataclass(frozen=True)
class QwenInspectionReport:
    """Decode-relevant fields of families/qwen.py:31-78 (inspect_qwen_hf_directory)."""

    model_dir: str
    model_type: str
    text_model_type: str | None
    has_vision_config: bool
    hidden_size: int
    head_dim: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    attn_output_gate: bool
    layer_types: list[str]
    full_attention_indices: list[int]
    supported_runtime: bool
    blocking_issues: list[str]


def inspect_qwen_hf_directory(model_dir: str | Path) -> QwenInspectionReport:
    """Read config.json and derive the decode geometry (families/qwen.py:265-353)."""
    root = Path(model_dir)
    config_path = root / "config.json"
    if not config_path.exists():
        raise FileNotFoundError(f"config.json not found in {root}")
    payload = json.loads(config_path.read_text(encoding="utf-8"))
    text_config = payload.get("text_config", payload)
    if not isinstance(text_config, dict):
        raise ValueError("Expected text_config to be a JSON object")
    vision_config = payload.get("vision_config")
    model_type = str(payload.get("model_type", ""))
    text_model_type = str(text_config["model_type"]) if text_config.get("model_type") is not None else None
    layer_types = [str(t) for t in text_config.get("layer_types", [])]
    full_attention = [i for i, t in enumerate(layer_types) if t == "full_attention"]
    head_dim = int(text_config["head_dim"])
    num_hidden_layers = int(text_config["num_hidden_layers"])
    num_attention_heads = int(text_config["num_attention_heads"])
    issues: list[str] = []
    if model_type not in SUPPORTED_QWEN_MODEL_TYPES:
        issues.append(f"Unsupported top-level model_type: {model_type}")
    if text_model_type is not None and text_model_type not in SUPPORTED_QWEN_MODEL_TYPES:
        issues.append(f"Unsupported text_config.model_type: {text_model_type}")
    if head_dim not in {64, 128, 256}:
        issues.append(f"Unsupported head_dim {head_dim}; torque-mlx currently supports only 64, 128, and 256")
    if len(layer_types) != num_hidden_layers:
        issues.append(f"layer_types length {len(layer_types)} does not match num_hidden_layers {num_hidden_layers}")
    if not full_attention:
        issues.append("No full_attention layers found; there is nothing to convert to TorqueKVCache")
    return QwenInspectionReport(
        model_dir=str(root.resolve()),
        model_type=model_type,
        text_model_type=text_model_type,
        has_vision_config=vision_config is not None,
        hidden_size=int(text_config.get("hidden_size", head_dim * num_attention_heads)),
        head_dim=head_dim,
        num_hidden_layers=num_hidden_layers,
        num_attention_heads=num_attention_heads,
        num_key_value_heads=int(text_config["num_key_value_heads"]),
        attn_output_gate=bool(text_config.get("attn_output_gate", False)),
        layer_types=layer_types,
        full_attention_indices=full_attention,
        supported_runtime=not issues,
        blocking_issues=issues,
    )


@dataclass(frozen=True)
class QwenModelArtifactManifest:
    """Decode-relevant fields of the converted-snapshot manifest (families/qwen.py:81-229): the runtime
    config, the converted layers and the two codebooks that `build_cache()` needs.  The conversion-only
    fields (tensor names, fusion modes, passthrough layers) are not read."""

    source_model_dir: str
    runtime_config: TorqueConfig
    converted_layer_indices: list[int]
    source_model_type: str
    source_text_model_type: str | None
    has_vision_config: bool
    key_codebook: Codebook
    value_codebook: Codebook


# Shorter name kept for callers of earlier versions of this package.
QwenModelManifest = QwenModelArtifactManifest


def load_qwen_model_manifest(model_dir: str | Path) -> QwenModelArtifactManifest:
    """families/qwen.py:414-418 (decode-relevant fields only)."""
    payload: Mapping[str, Any] = json.loads((Path(model_dir) / QWEN_MODEL_MANIFEST_FILE).read_text(encoding="utf-8"))
    return QwenModelArtifactManifest(
        source_model_dir=str(payload["source_model_dir"]),
        runtime_config=config_from_dict(dict(payload["runtime_config"])),
        converted_layer_indices=[int(i) for i in payload["converted_layer_indices"]],
        source_model_type=str(payload["source_model_type"]),
        source_text_model_type=(
            str(payload["source_text_model_type"]) if payload.get("source_text_model_type") is not None else None
        ),
        has_vision_config=bool(payload.get("has_vision_config", False)),
        key_codebook=Codebook.from_dict(dict(payload["key_codebook"])),
        value_codebook=Codebook.from_dict(dict(payload["value_codebook"])),
    )


def _fp16_kv_bytes_per_token(*, head_dim: int, kv_heads: int) -> int:
    return head_dim * kv_heads * 2 * 2


@dataclass(frozen=True)
class QwenDecodeBenchmarkProfile:
    model_dir: str
    profile_source: str
    model_type: str
    text_model_type: str | None
    hidden_size: int | None
    head_dim: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    target_layer_indices: tuple[int, ...]
    bit_width: int
    rotation_seed: int
    fused_weights: bool
    has_vision_config: bool
    attn_output_gate: bool

    @property
    def target_layer_count(self) -> int:
        return len(self.target_layer_indices)

    @property
    def kv_group_ratio(self) -> float:
        return float(self.num_attention_heads) / float(self.num_key_value_heads)

    @property
    def torque_kv_bytes_per_token_per_layer(self) -> int:
        return kv_bytes_per_token(head_dim=self.head_dim, bit_width=self.bit_width, kv_heads=self.num_key_value_heads)

    @property
    def fp16_kv_bytes_per_token_per_layer(self) -> int:
        return _fp16_kv_bytes_per_token(head_dim=self.head_dim, kv_heads=self.num_key_value_heads)

    def to_dict(self) -> dict[str, object]:
        """Keys of qwen_benchmark.py:81-105."""
        return {
            "family": "qwen",
            "model_dir": self.model_dir,
            "profile_source": self.profile_source,
            "model_type": self.model_type,
            "text_model_type": self.text_model_type,
            "hidden_size": self.hidden_size,
            "head_dim": self.head_dim,
            "num_hidden_layers": self.num_hidden_layers,
            "num_attention_heads": self.num_attention_heads,
            "num_key_value_heads": self.num_key_value_heads,
            "kv_group_ratio": self.kv_group_ratio,
            "target_layer_indices": list(self.target_layer_indices),
            "target_layer_count": self.target_layer_count,
            "bit_width": self.bit_width,
            "rotation_seed": self.rotation_seed,
            "fused_weights": self.fused_weights,
            "has_vision_config": self.has_vision_config,
            "attn_output_gate": self.attn_output_gate,
            "fp16_kv_bytes_per_token_per_layer": self.fp16_kv_bytes_per_token_per_layer,
            "torque_kv_bytes_per_token_per_layer": self.torque_kv_bytes_per_token_per_layer,
            "fp16_kv_bytes_per_token_total": self.fp16_kv_bytes_per_token_per_layer * self.target_layer_count,
            "torque_kv_bytes_per_token_total": self.torque_kv_bytes_per_token_per_layer * self.target_layer_count,
        }


@dataclass(frozen=True)
class QwenDecodeRuntimeBenchmarkResult:
    profile: QwenDecodeBenchmarkProfile
    prefill_tokens: int
    decode_steps: int
    seed: int
    torque_decode_strategy: str
    torque_decode_tail_capacity: int
    fp16_update_seconds: float
    fp16_attention_seconds: float
    fp16_decode_seconds: float
    mlx_lm_quantized_update_seconds: float | None
    mlx_lm_quantized_attention_seconds: float | None
    mlx_lm_quantized_decode_seconds: float | None
    torque_append_seconds: float
    torque_kernel_seconds: float
    torque_decode_seconds: float
    max_abs_error_quantized_vs_fp16: float | None
    max_abs_error_torque_vs_fp16: float

    def to_dict(self) -> dict[str, object]:
        """Keys of qwen_benchmark.py:128-176, plus explicit fp16-dense keys."""
        total_tokens = self.prefill_tokens + self.decode_steps
        layers = self.profile.target_layer_count
        fp16_total = self.profile.fp16_kv_bytes_per_token_per_layer * layers * total_tokens
        torque_total = self.profile.torque_kv_bytes_per_token_per_layer * layers * total_tokens

        def host(total: float, *parts: float) -> float:
            return max(0.0, total - sum(parts))

        def tps(seconds: float) -> float:
            return self.decode_steps / seconds if seconds > 0 else 0.0

        def ms(seconds: float | None) -> float | None:
            return None if seconds is None else seconds * 1_000.0

        # MLX-LM's quantized comparator does not exist on this backend: its figures are reported as null.
        quantized_absent = self.mlx_lm_quantized_decode_seconds is None

        fp16 = {
            "update_ms": self.fp16_update_seconds * 1_000.0,
            "attention_ms": self.fp16_attention_seconds * 1_000.0,
            "host_overhead_ms": host(self.fp16_decode_seconds, self.fp16_update_seconds, self.fp16_attention_seconds) * 1_000.0,
            "decode_ms": self.fp16_decode_seconds * 1_000.0,
            "tokens_per_sec": tps(self.fp16_decode_seconds),
        }
        payload: dict[str, object] = {
            "family": "qwen",
            "benchmark": "qwen_decode_runtime",
            "profile": self.profile.to_dict(),
            "prefill_tokens": self.prefill_tokens,
            "decode_steps": self.decode_steps,
            "seed": self.seed,
            "torque_decode_strategy": self.torque_decode_strategy,
            "torque_decode_tail_capacity": self.torque_decode_tail_capacity,
            "notes": [
                "This benchmark measures the KV-growing decode hot path only, not full dense forwards or perplexity.",
                "It uses the Qwen model geometry from the local snapshot or torque manifest.",
                "Backend: HIP on MI355X. mlx_fp16_* report the fp16-dense HIP decode kernel; "
                "MLX-LM's QuantizedKVCache has no counterpart: mlx_lm_quantized_* and "
                "max_abs_error_quantized_vs_fp16 are null.",
            ],
            "fp16_kv_cache_total_bytes": fp16_total,
            "torque_kv_cache_total_bytes": torque_total,
            "fp16_kv_cache_total_gib": fp16_total / float(1 << 30),
            "torque_kv_cache_total_gib": torque_total / float(1 << 30),
            "kv_cache_bytes_saved_vs_fp16": fp16_total - torque_total,
            "mlx_lm_quantized_update_ms": ms(self.mlx_lm_quantized_update_seconds),
            "mlx_lm_quantized_attention_ms": ms(self.mlx_lm_quantized_attention_seconds),
            "mlx_lm_quantized_host_overhead_ms": None if quantized_absent else host(
                self.mlx_lm_quantized_decode_seconds,
                self.mlx_lm_quantized_update_seconds,
                self.mlx_lm_quantized_attention_seconds,
            ) * 1_000.0,
            "mlx_lm_quantized_decode_ms": ms(self.mlx_lm_quantized_decode_seconds),
            "mlx_lm_quantized_tokens_per_sec": None if quantized_absent else tps(self.mlx_lm_quantized_decode_seconds),
            "torque_mlx_append_ms": self.torque_append_seconds * 1_000.0,
            "torque_mlx_kernel_ms": self.torque_kernel_seconds * 1_000.0,
            "torque_mlx_host_overhead_ms": host(
                self.torque_decode_seconds, self.torque_append_seconds, self.torque_kernel_seconds
            ) * 1_000.0,
            "torque_mlx_decode_ms": self.torque_decode_seconds * 1_000.0,
            "torque_mlx_tokens_per_sec": tps(self.torque_decode_seconds),
            "max_abs_error_quantized_vs_fp16": self.max_abs_error_quantized_vs_fp16,
            "max_abs_error_torque_vs_fp16": self.max_abs_error_torque_vs_fp16,
        }
        for key, value in fp16.items():
            payload[f"mlx_fp16_{key}"] = value
            payload[f"fp16_dense_{key}"] = value
        return payload


def load_qwen_decode_benchmark_profile(
    model_dir: str | Path,
    *,
    bit_width: int | None = None,
    rotation_seed: int = 0,
    fused_weights: bool = False,
) -> QwenDecodeBenchmarkProfile:
    """Profile from a converted manifest or an HF snapshot (qwen_benchmark.py:212-271)."""
    root = Path(model_dir)
    if (root / QWEN_MODEL_MANIFEST_FILE).exists():
        manifest = load_qwen_model_manifest(root)
        source_root = Path(manifest.source_model_dir)
        report = inspect_qwen_hf_directory(source_root) if source_root.exists() else None
        return QwenDecodeBenchmarkProfile(
            model_dir=str(root.resolve()),
            profile_source="torque_manifest",
            model_type=manifest.source_model_type,
            text_model_type=manifest.source_text_model_type,
            hidden_size=report.hidden_size if report is not None else None,
            head_dim=manifest.runtime_config.head_dim,
            num_hidden_layers=manifest.runtime_config.num_layers,
            num_attention_heads=report.num_attention_heads if report is not None else manifest.runtime_config.kv_heads,
            num_key_value_heads=manifest.runtime_config.kv_heads,
            target_layer_indices=tuple(manifest.converted_layer_indices),
            bit_width=manifest.runtime_config.bit_width,
            rotation_seed=manifest.runtime_config.rotation_seed,
            fused_weights=fused_weights,
            has_vision_config=manifest.has_vision_config,
            attn_output_gate=report.attn_output_gate if report is not None else False,
        )
    report = inspect_qwen_hf_directory(root)
    if not report.supported_runtime:
        raise ValueError("Qwen model is not currently supported by torque-mlx: " + "; ".join(report.blocking_issues))
    return QwenDecodeBenchmarkProfile(
        model_dir=str(root.resolve()),
        profile_source="hf_snapshot",
        model_type=report.model_type,
        text_model_type=report.text_model_type,
        hidden_size=report.hidden_size,
        head_dim=report.head_dim,
        num_hidden_layers=report.num_hidden_layers,
        num_attention_heads=report.num_attention_heads,
        num_key_value_heads=report.num_key_value_heads,
        target_layer_indices=tuple(report.full_attention_indices),
        bit_width=4 if bit_width is None else bit_width,
        rotation_seed=rotation_seed,
        fused_weights=fused_weights,
        has_vision_config=report.has_vision_config,
        attn_output_gate=report.attn_output_gate,
    )


def _build_decode_inputs(*, profile: QwenDecodeBenchmarkProfile, prefill_tokens: int, decode_steps: int, seed: int):
    """uniform(-1, 1) K/V [Lt, 1, Hkv, P+N, D] and Q [Lt, 1, Hq, N, D] (qwen_benchmark.py:274-297)."""
    rng = np.random.default_rng(seed)
    total = prefill_tokens + decode_steps
    shape = (profile.target_layer_count, 1, profile.num_key_value_heads, total, profile.head_dim)
    keys = rng.uniform(-1.0, 1.0, size=shape).astype(np.float32)
    values = rng.uniform(-1.0, 1.0, size=shape).astype(np.float32)
    queries = rng.uniform(
        -1.0, 1.0, size=(profile.target_layer_count, 1, profile.num_attention_heads, decode_steps, profile.head_dim)
    ).astype(np.float32)
    return keys, values, queries


def _sync_time(fn) -> float:
    torch.cuda.synchronize()
    started = perf_counter()
    fn()
    torch.cuda.synchronize()
    return perf_counter() - started


def _run_qwen_decode_runtime_benchmark_impl(
    *,
    profile: QwenDecodeBenchmarkProfile,
    prefill_tokens: int,
    decode_steps: int,
    seed: int,
    decode_strategy: str,
    decode_tail_capacity: int,
) -> QwenDecodeRuntimeBenchmarkResult:
    """The KV-growing decode loop of qwen_benchmark.py:300-454 on the HIP path."""
    if prefill_tokens <= 0:
        raise ValueError("prefill_tokens must be positive")
    if decode_steps <= 0:
        raise ValueError("decode_steps must be positive")
    if profile.target_layer_count <= 0:
        raise ValueError("Qwen decode benchmark requires at least one target layer")
    dev = device()
    keys_np, values_np, queries_np = _build_decode_inputs(
        profile=profile, prefill_tokens=prefill_tokens, decode_steps=decode_steps, seed=seed
    )
    lt, hkv, hq, d = profile.target_layer_count, profile.num_key_value_heads, profile.num_attention_heads, profile.head_dim
    total = prefill_tokens + decode_steps
    keys = torch.from_numpy(keys_np[:, 0]).to(dev)      # [Lt, Hkv, total, D]
    values = torch.from_numpy(values_np[:, 0]).to(dev)
    queries = torch.from_numpy(queries_np[:, 0]).to(dev)  # [Lt, Hq, N, D]

    # fp16-dense comparator: slab [Lt, Hkv, total, D] updated in place each step.
    k16 = torch.zeros((lt, hkv, total, d), dtype=torch.float16, device=dev)
    v16 = torch.zeros_like(k16)
    k16[:, :, :prefill_tokens] = keys[:, :, :prefill_tokens].half()
    v16[:, :, :prefill_tokens] = values[:, :, :prefill_tokens].half()
    fp16_out = torch.empty((lt, hq, d), dtype=torch.float32, device=dev)
    fp16_update = fp16_attention = 0.0
    started = perf_counter()
    for step in range(decode_steps):
        pos = prefill_tokens + step
        fp16_update += _sync_time(lambda: (k16[:, :, pos].copy_(keys[:, :, pos]), v16[:, :, pos].copy_(values[:, :, pos])))
        q_step = queries[:, :, step].contiguous()
        fp16_attention += _sync_time(
            lambda: ops.dense_decode(
                q_step, k16, v16, num_layers=lt, query_heads=hq, kv_heads=hkv, head_dim=d,
                capacity=total, seq_len=pos + 1, out=fp16_out,
            )
        )
    torch.cuda.synchronize()
    fp16_elapsed = perf_counter() - started
    fp16_final = fp16_out.cpu().numpy()

    cache = TorqueKVCacheHIP(
        config=TorqueConfig(
            bit_width=profile.bit_width,
            head_dim=d,
            num_layers=lt,
            kv_heads=hkv,
            fused_weights=profile.fused_weights,
            rotation_seed=profile.rotation_seed,
        ),
        key_codebook=build_uniform_codebook(profile.bit_width),
        value_codebook=build_uniform_codebook(profile.bit_width),
        initial_capacity=total,
        decode_strategy=decode_strategy,
        decode_tail_capacity=decode_tail_capacity,
    )
    cache.append_many(key=keys[:, :, :prefill_tokens], value=values[:, :, :prefill_tokens])
    torch.cuda.synchronize()
    append_elapsed = kernel_elapsed = 0.0
    torque_out = None
    started = perf_counter()
    for step in range(decode_steps):
        pos = prefill_tokens + step
        t0 = perf_counter()
        cache.append(key=keys_np[:, 0, :, pos, :], value=values_np[:, 0, :, pos, :])
        torch.cuda.synchronize()
        append_elapsed += perf_counter() - t0
        t0 = perf_counter()
        torque_out = cache.decode(query=queries_np[:, 0, :, step, :], return_numpy=False)
        torch.cuda.synchronize()
        kernel_elapsed += perf_counter() - t0
        torque_final = torque_out.cpu().numpy()
    torque_elapsed = perf_counter() - started

    return QwenDecodeRuntimeBenchmarkResult(
        profile=profile,
        prefill_tokens=prefill_tokens,
        decode_steps=decode_steps,
        seed=seed,
        torque_decode_strategy=decode_strategy,
        torque_decode_tail_capacity=decode_tail_capacity,
        fp16_update_seconds=fp16_update,
        fp16_attention_seconds=fp16_attention,
        fp16_decode_seconds=fp16_elapsed,
        mlx_lm_quantized_update_seconds=None,
        mlx_lm_quantized_attention_seconds=None,
        mlx_lm_quantized_decode_seconds=None,
        torque_append_seconds=append_elapsed,
        torque_kernel_seconds=kernel_elapsed,
        torque_decode_seconds=torque_elapsed,
        max_abs_error_quantized_vs_fp16=None,
        max_abs_error_torque_vs_fp16=float(np.max(np.abs(torque_final - fp16_final))),
    )


def run_qwen_decode_runtime_benchmark(
    *,
    model_dir: str | Path,
    prefill_tokens: int,
    decode_steps: int,
    seed: int,
    bit_width: int | None = None,
    rotation_seed: int = 0,
    fused_weights: bool = False,
    decode_strategy: str = "split_batched",
    decode_tail_capacity: int | None = None,
    runner: Callable[..., QwenDecodeRuntimeBenchmarkResult] | None = None,
) -> QwenDecodeRuntimeBenchmarkResult:
    """Entry point with runner injection (qwen_benchmark.py:457-493)."""
    if decode_strategy not in SUPPORTED_DECODE_STRATEGIES:
        raise ValueError("decode_strategy must be one of " + ", ".join(SUPPORTED_DECODE_STRATEGIES))
    profile = load_qwen_decode_benchmark_profile(
        model_dir, bit_width=bit_width, rotation_seed=rotation_seed, fused_weights=fused_weights
    )
    runtime_runner = runner or _run_qwen_decode_runtime_benchmark_impl
    return runtime_runner(
        profile=profile,
        prefill_tokens=prefill_tokens,
        decode_steps=decode_steps,
        seed=seed,
        decode_strategy=decode_strategy,
        decode_tail_capacity=resolve_qwen_decode_tail_capacity(hidden_size=profile.hidden_size, requested=decode_tail_capacity),
    )

"""Harness logic without a GPU, mirroring the reference's tests/test_qwen_benchmark.py
(profile loading from config.json / manifest, runner injection, CLI dispatch)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from torque_hip import cli
from torque_hip.qwen_benchmark import (
    QWEN_MODEL_MANIFEST_FILE,
    QwenDecodeBenchmarkProfile,
    QwenDecodeRuntimeBenchmarkResult,
    load_qwen_decode_benchmark_profile,
    resolve_qwen_decode_tail_capacity,
    run_qwen_decode_runtime_benchmark,
)


def _write_qwen_config(model_dir: Path, **overrides) -> None:
    # test_qwen_benchmark.py:23-43
    text = {
        "model_type": "qwen3_5",
        "hidden_size": 1024,
        "head_dim": 256,
        "num_hidden_layers": 4,
        "num_attention_heads": 8,
        "num_key_value_heads": 2,
        "attn_output_gate": True,
        "layer_types": ["linear_attention", "linear_attention", "linear_attention", "full_attention"],
    }
    text.update(overrides)
    payload = {"architectures": ["Qwen3_5ForCausalLM"], "model_type": "qwen3_5", "text_config": text}
    (model_dir / "config.json").write_text(json.dumps(payload), encoding="utf-8")


def _write_manifest(model_dir: Path, source_model_dir: Path) -> None:
    # test_qwen_benchmark.py:46-75
    cb = {"bit_width": 4, "centroids": np.linspace(-1.0, 1.0, 16).tolist(), "name": "gaussian"}
    payload = {
        "model_name": "qwen-benchmark-test",
        "source_model_dir": str(source_model_dir),
        "runtime_config": {"bit_width": 4, "head_dim": 256, "num_layers": 4, "kv_heads": 2, "fused_weights": True,
                           "rotation_mode": "hadamard", "rotation_seed": 7},
        "full_attention_indices": [3],
        "converted_layer_indices": [3],
        "passthrough_layer_indices": [0, 1, 2],
        "converted_tensor_names": {"3": []},
        "key_codebook": cb,
        "value_codebook": cb,
        "source_model_type": "qwen3_5",
        "source_text_model_type": "qwen3_5",
        "source_vision_model_type": None,
        "has_vision_config": False,
        "source_architectures": ["Qwen3_5ForCausalLM"],
    }
    (model_dir / QWEN_MODEL_MANIFEST_FILE).write_text(json.dumps(payload), encoding="utf-8")


def test_profile_from_source_snapshot(tmp_path):
    # test_qwen_benchmark.py:78-94
    _write_qwen_config(tmp_path)
    profile = load_qwen_decode_benchmark_profile(tmp_path, bit_width=3, rotation_seed=11)
    assert profile.profile_source == "hf_snapshot"
    assert profile.hidden_size == 1024 and profile.head_dim == 256
    assert profile.num_attention_heads == 8 and profile.num_key_value_heads == 2
    assert profile.target_layer_indices == (3,) and profile.bit_width == 3 and profile.rotation_seed == 11
    assert profile.kv_group_ratio == 4.0
    assert profile.to_dict()["torque_kv_bytes_per_token_per_layer"] == 2 * 24 * 4 * 2


def test_profile_from_manifest_recovers_source_geometry(tmp_path):
    # test_qwen_benchmark.py:97-114
    source = tmp_path / "source"
    source.mkdir()
    _write_qwen_config(source)
    artifact = tmp_path / "torque"
    artifact.mkdir()
    _write_manifest(artifact, source)
    profile = load_qwen_decode_benchmark_profile(artifact)
    assert profile.profile_source == "torque_manifest"
    assert profile.hidden_size == 1024 and profile.num_attention_heads == 8 and profile.num_key_value_heads == 2
    assert profile.bit_width == 4 and profile.rotation_seed == 7 and profile.target_layer_indices == (3,)


def test_unsupported_snapshot_is_rejected(tmp_path):
    _write_qwen_config(tmp_path, head_dim=96)
    with pytest.raises(ValueError, match="Unsupported head_dim 96"):
        load_qwen_decode_benchmark_profile(tmp_path)


def test_tail_capacity_heuristic():
    # qwen_mlx.py:18-30
    assert resolve_qwen_decode_tail_capacity(hidden_size=1024, requested=None) == 8
    assert resolve_qwen_decode_tail_capacity(hidden_size=4096, requested=None) == 0
    assert resolve_qwen_decode_tail_capacity(hidden_size=None, requested=None) == 8
    assert resolve_qwen_decode_tail_capacity(hidden_size=4096, requested=96) == 96


def _fake_result(profile, **kw):
    base = dict(
        profile=profile, prefill_tokens=128, decode_steps=16, seed=3, torque_decode_strategy="split_batched",
        torque_decode_tail_capacity=8, fp16_update_seconds=0.2, fp16_attention_seconds=0.3, fp16_decode_seconds=1.0,
        mlx_lm_quantized_update_seconds=0.4, mlx_lm_quantized_attention_seconds=0.5,
        mlx_lm_quantized_decode_seconds=2.0, torque_append_seconds=0.1, torque_kernel_seconds=0.2,
        torque_decode_seconds=0.5, max_abs_error_quantized_vs_fp16=0.1, max_abs_error_torque_vs_fp16=0.2,
    )
    base.update(kw)
    return QwenDecodeRuntimeBenchmarkResult(**base)


def test_runner_injection(tmp_path):
    # test_qwen_benchmark.py:117-163
    _write_qwen_config(tmp_path)

    def fake_runner(**kwargs):
        assert kwargs["profile"].target_layer_count == 1
        assert kwargs["prefill_tokens"] == 128 and kwargs["decode_steps"] == 16
        assert kwargs["decode_tail_capacity"] == 8
        return _fake_result(kwargs["profile"], torque_decode_strategy=kwargs["decode_strategy"])

    payload = run_qwen_decode_runtime_benchmark(
        model_dir=tmp_path, prefill_tokens=128, decode_steps=16, seed=3, bit_width=4, runner=fake_runner
    ).to_dict()
    assert payload["benchmark"] == "qwen_decode_runtime"
    assert payload["profile"]["target_layer_count"] == 1
    assert payload["torque_decode_strategy"] == "split_batched"
    assert payload["torque_decode_tail_capacity"] == 8
    assert payload["torque_mlx_tokens_per_sec"] == 32.0
    assert payload["torque_mlx_append_ms"] == 100.0
    assert payload["fp16_dense_attention_ms"] == payload["mlx_fp16_attention_ms"] == 300.0
    with pytest.raises(ValueError, match="decode_strategy must be one of"):
        run_qwen_decode_runtime_benchmark(model_dir=tmp_path, prefill_tokens=1, decode_steps=1, seed=0,
                                          decode_strategy="bogus", runner=fake_runner)


def test_cli_qwen_decode_dispatch(monkeypatch, capsys, tmp_path):
    # test_qwen_benchmark.py:166-234
    profile = QwenDecodeBenchmarkProfile(
        model_dir=str(tmp_path), profile_source="hf_snapshot", model_type="qwen3_5", text_model_type="qwen3_5",
        hidden_size=1024, head_dim=256, num_hidden_layers=4, num_attention_heads=8, num_key_value_heads=2,
        target_layer_indices=(3,), bit_width=4, rotation_seed=0, fused_weights=False, has_vision_config=False,
        attn_output_gate=True,
    )

    def fake_benchmark(**kwargs):
        assert kwargs["model_dir"] == str(tmp_path)
        assert kwargs["prefill_tokens"] == 256 and kwargs["decode_steps"] == 32
        assert kwargs["decode_tail_capacity"] is None
        return _fake_result(profile, prefill_tokens=256, decode_steps=32, torque_decode_strategy=kwargs["decode_strategy"])

    monkeypatch.setattr("torque_hip.cli.run_qwen_decode_runtime_benchmark", fake_benchmark)
    rc = cli.main(["benchmark", "qwen-decode", "--model-dir", str(tmp_path), "--prefill-tokens", "256",
                   "--decode-steps", "32", "--decode-strategy", "split_batched"])
    assert rc == 0
    payload = json.loads(capsys.readouterr().out)
    assert payload["benchmark"] == "qwen_decode_runtime" and payload["torque_decode_strategy"] == "split_batched"


def test_cli_parser():
    # test_qwen_benchmark.py:237-255; cli.py:65-74 defaults
    args = cli.build_parser().parse_args(["benchmark", "qwen-decode", "--model-dir", "./a", "--prefill-tokens", "128",
                                          "--decode-steps", "16", "--decode-tail-capacity", "96"])
    assert args.benchmark_command == "qwen-decode" and args.decode_tail_capacity == 96
    syn = cli.build_parser().parse_args(["benchmark", "synthetic"])
    assert (syn.seq_len, syn.head_dim, syn.kv_heads, syn.bit_width, syn.seed) == (512, 128, 8, 4, 0)


def test_bench_reads_committed_traffic_and_refuses_multi_gpu():
    import importlib.util
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    spec = importlib.util.spec_from_file_location("bench_under_test", root / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    traffic, src = bench.measured_traffic("decode_kernel<PackedB4,128,4>", "M")
    assert src and src.startswith("profiles/") and 32 * 2**20 <= traffic <= 40 * 2**20
    assert bench.measured_traffic("decode_kernel<PackedB4,128,4>", "no-such-workload") == (None, None)
    proc = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert proc.returncode == 2 and "one GPU" in proc.stderr

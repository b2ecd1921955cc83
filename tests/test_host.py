"""Host-side logic of the torque_hip package (no GPU): configuration, layout,
codebooks, artifact manifests and constructor validation."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import torque_hip as th
from torque_hip.cache_hip import TorqueKVCacheHIP

GOLDEN = Path(__file__).with_name("golden")


def test_config_validation_and_variant():
    assert th.TorqueConfig(bit_width=3, head_dim=128, fused_weights=True).variant_id == "b3-h128-hadamard-fused"
    assert th.TorqueConfig().variant_id == "b4-h128-hadamard-unfused"
    for bad, msg in ((dict(bit_width=5), "Unsupported bit width"), (dict(head_dim=96), "Unsupported head dimension"),
                     (dict(num_layers=0), "num_layers"), (dict(kv_heads=0), "kv_heads"),
                     (dict(scale_mode="max"), "scale_mode")):
        with pytest.raises(ValueError, match=msg):
            th.TorqueConfig(**bad).validate()


def test_scale_mode_config_and_manifest_fields():
    """The per-vector scale extension: reference-format manifests carry no scale_mode field and load as "none";
    "rms" round-trips and marks the variant id."""
    from torque_hip.artifact import config_from_dict, config_to_dict

    plain = th.TorqueConfig(bit_width=4, head_dim=128, kv_heads=8)
    assert "scale_mode" not in config_to_dict(plain) and config_from_dict(config_to_dict(plain)) == plain
    rms = th.TorqueConfig(bit_width=4, head_dim=128, kv_heads=8, scale_mode="rms")
    assert config_to_dict(rms)["scale_mode"] == "rms" and config_from_dict(config_to_dict(rms)) == rms
    assert rms.variant_id == "b4-h128-hadamard-unfused-rms"


def test_layout():
    lay = th.PackedKVLayout(bit_width=3, head_dim=64)
    assert (lay.packed_words, lay.packed_bytes, lay.kv_bytes_per_token_per_head) == (6, 24, 48)
    assert lay.tensor_shape(num_layers=2, kv_heads=4, seq_len=9) == (2, 4, 9, 6)
    assert th.kv_bytes_per_token(128, 4, 8) == 16 * 4 * 8 * 2


def test_codebook_json_roundtrip(tmp_path):
    # test_quantization.py:114-121
    from torque_hip.quantization import load_codebook, save_codebook

    cb = th.build_gaussian_codebook(4, sample_size=20_000, iterations=12, seed=7)
    path = tmp_path / "codebook.json"
    save_codebook(cb, path)
    loaded = load_codebook(path)
    assert loaded.bit_width == cb.bit_width and loaded.name == cb.name
    np.testing.assert_array_equal(loaded.centroids, cb.centroids)


def test_codebook_validation():
    with pytest.raises(ValueError, match="Expected 4 centroids"):
        th.Codebook(bit_width=2, centroids=np.zeros(3))
    with pytest.raises(ValueError, match="sorted"):
        th.Codebook(bit_width=2, centroids=np.array([1.0, 0.0, 2.0, 3.0]))


def test_package_codebook_builder_matches_reference_goldens():
    payload = json.loads((GOLDEN / "gaussian_codebooks.json").read_text())
    for case in payload["cases"]:
        expected = np.array([int(h, 16) for h in case["centroids_hex"]], dtype=np.uint32).view(np.float32)
        cb = th.build_gaussian_codebook(case["bit_width"], seed=case["seed"], sample_size=case["sample_size"],
                                        iterations=case["iterations"])
        np.testing.assert_array_equal(cb.centroids, expected)
        bnd = np.array([int(h, 16) for h in case["boundaries_hex"]], dtype=np.uint32).view(np.float32)
        np.testing.assert_array_equal(th.codebook_boundaries(cb), bnd)


def test_rotation_signs_follow_reference_rng():
    from oracle import torque_oracle as o

    for d in (64, 128, 256):
        spec = th.RotationSpec.from_seed(d, 13)
        sl, sr = o.rotation_signs_from_seed(d, 13)
        np.testing.assert_array_equal(spec.signs_left, sl)
        np.testing.assert_array_equal(spec.signs_right, sr)
    with pytest.raises(ValueError, match="Unsupported head dimension"):
        th.RotationSpec.from_seed(100)
    with pytest.raises(ValueError, match="must match head_dim"):
        th.RotationSpec(head_dim=64, signs_left=np.ones(64), signs_right=np.ones(32))


def test_cache_constructor_validation():
    cfg = th.TorqueConfig(bit_width=4, head_dim=64)
    for bad, msg in ((dict(initial_capacity=0), "initial_capacity"), (dict(growth_factor=1), "growth_factor"),
                     (dict(decode_tail_capacity=-1), "decode_tail_capacity"), (dict(decode_strategy="x"), "decode_strategy")):
        with pytest.raises(ValueError, match=msg):
            TorqueKVCacheHIP(config=cfg, **bad)
    assert th.SUPPORTED_DECODE_STRATEGIES == ("auto", "split_batched", "fused_per_head")
    assert th.TorqueKVCacheMLX is TorqueKVCacheHIP


def _manifest_payload(**overrides):
    cb = th.build_uniform_codebook(4).to_dict()
    payload = {
        "model_name": "m",
        "architecture": "generic_decoder_attention",
        "source_format": "numpy_npz",
        "runtime_config": {"bit_width": 4, "head_dim": 64, "num_layers": 2, "kv_heads": 2, "fused_weights": True,
                           "rotation_mode": "hadamard", "rotation_seed": 5},
        "key_codebook": cb,
        "value_codebook": cb,
    }
    payload.update(overrides)
    return payload


def test_artifact_manifest_roundtrip_and_load(tmp_path):
    from torque_hip.artifact import TorqueArtifactManifest

    manifest = TorqueArtifactManifest.from_dict(_manifest_payload())
    again = TorqueArtifactManifest.from_dict(json.loads(json.dumps(manifest.to_dict())))
    assert again.to_dict() == manifest.to_dict()
    assert manifest.to_dict()["variant_id"] == "b4-h64-hadamard-fused"
    (tmp_path / "manifest.json").write_text(json.dumps(manifest.to_dict()))
    w = np.zeros((64, 8), dtype=np.float32)
    np.savez(tmp_path / "weights.npz", w_q=w, w_k=w, w_v=w, w_o=np.zeros((8, 64), np.float32))
    art = th.load_torque_artifact(tmp_path)
    assert art.runtime_config.rotation_seed == 5 and art.fused_weights.w_o.shape == (8, 64)


def test_artifact_manifest_errors():
    from torque_hip.artifact import TorqueArtifactManifest

    with pytest.raises(ValueError, match="Missing required fields"):
        TorqueArtifactManifest.from_dict({"model_name": "m"})
    bad = _manifest_payload()
    bad["runtime_config"] = dict(bad["runtime_config"], fused_weights=False)
    with pytest.raises(ValueError, match="fused_weights"):
        TorqueArtifactManifest.from_dict(bad)
    with pytest.raises(ValueError, match="Unsupported artifact version"):
        TorqueArtifactManifest.from_dict(_manifest_payload(format_version=2))


# The reference package's public names (src/torque_mlx/__init__.py:38-68), split by
# whether they sit on the packed decode path this package replaces.
REFERENCE_EXPORTS_IN_SCOPE = (
    "QwenDecodeBenchmarkProfile",  # qwen_benchmark.py:40-105
    "QwenDecodeRuntimeBenchmarkResult",  # qwen_benchmark.py:128-176
    "QwenInspectionReport",  # families/qwen.py:31-78 (read by the qwen-decode profile loader)
    "QwenModelArtifactManifest",  # families/qwen.py:81-229 (the manifest feeding build_cache)
    "TorqueArtifact",
    "TorqueArtifactManifest",
    "TorqueConfig",
    "TorqueKVCache",
    "TorqueKVCacheMLX",
    "decode_packed_attention",
    "inspect_qwen_hf_directory",
    "load_qwen_decode_benchmark_profile",
    "load_qwen_model_manifest",
    "load_torque_artifact",
    "metal_available",
    "run_qwen_decode_runtime_benchmark",
    "run_synthetic_decode_benchmark",
)
# Conversion, weight fusion, Qwen text evaluation and artifact writing: not on the decode path,
# deliberately absent.
REFERENCE_EXPORTS_OUT_OF_SCOPE = (
    "FusedAttentionWeights",
    "QwenTextBenchmarkCase",
    "QwenTextBenchmarkComparison",
    "QwenTextPerplexityResult",
    "benchmark_qwen_text_models",
    "build_torque_artifact",
    "convert_npz_checkpoint",
    "convert_qwen_attention_layer",
    "convert_qwen_model",
    "evaluate_artifact",
    "evaluate_qwen_text_perplexity",
    "fuse_attention_weights",
)


def test_reference_exports_resolve():
    """`import torque_hip as torque_mlx` resolves every decode-path name of the reference's __all__."""
    assert len(REFERENCE_EXPORTS_IN_SCOPE) + len(REFERENCE_EXPORTS_OUT_OF_SCOPE) == 29
    for name in REFERENCE_EXPORTS_IN_SCOPE:
        assert hasattr(th, name), name
        assert name in th.__all__, name
    for name in REFERENCE_EXPORTS_OUT_OF_SCOPE:
        assert not hasattr(th, name), name
    assert callable(th.run_synthetic_decode_benchmark) and callable(th.run_qwen_decode_runtime_benchmark)

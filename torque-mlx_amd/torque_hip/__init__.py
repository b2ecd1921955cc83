"""torque_hip -- MI355X-native packed rotated KV-cache decode path.

Drop-in for the decode hot path of cbun/torque-mlx: the same cache classes,
operator wrappers and benchmark harnesses, with every computation in
hand-written HIP kernels for gfx950 behind the C ABI in include/torque_hip.h.
"""

from torque_hip._lib import hip_available
from torque_hip.artifact import TorqueArtifact, TorqueArtifactManifest, load_torque_artifact
from torque_hip.benchmarking import run_synthetic_decode_benchmark
from torque_hip.cache import TorqueKVCache
from torque_hip.cache_hip import SUPPORTED_DECODE_STRATEGIES, TorqueKVCacheHIP, TorqueKVCacheMLX
from torque_hip.config import TorqueConfig
from torque_hip.layout import CacheMetadata, PackedKVLayout, build_variant_id
from torque_hip.ops import (
    decode_packed_attention,
    decode_packed_attention_split,
    decode_packed_attention_split_batched,
    decode_packed_attention_split_batched_with_current,
    metal_available,
    quantize_and_pack_rows,
    quantize_and_pack_rows_dual,
)
from torque_hip.qwen_benchmark import (
    QwenDecodeBenchmarkProfile,
    QwenDecodeRuntimeBenchmarkResult,
    QwenInspectionReport,
    QwenModelArtifactManifest,
    inspect_qwen_hf_directory,
    load_qwen_decode_benchmark_profile,
    load_qwen_model_manifest,
    run_qwen_decode_runtime_benchmark,
)
from torque_hip.quantization import (
    Codebook,
    build_gaussian_codebook,
    build_uniform_codebook,
    codebook_boundaries,
    kv_bytes_per_token,
    packed_words_for_head_dim,
)
from torque_hip.rotation import RotationMode, RotationSpec

__all__ = [
    "CacheMetadata",
    "Codebook",
    "PackedKVLayout",
    "QwenDecodeBenchmarkProfile",
    "QwenDecodeRuntimeBenchmarkResult",
    "QwenInspectionReport",
    "QwenModelArtifactManifest",
    "RotationMode",
    "RotationSpec",
    "SUPPORTED_DECODE_STRATEGIES",
    "TorqueArtifact",
    "TorqueArtifactManifest",
    "TorqueConfig",
    "TorqueKVCache",
    "TorqueKVCacheHIP",
    "TorqueKVCacheMLX",
    "build_gaussian_codebook",
    "build_uniform_codebook",
    "build_variant_id",
    "codebook_boundaries",
    "decode_packed_attention",
    "decode_packed_attention_split",
    "decode_packed_attention_split_batched",
    "decode_packed_attention_split_batched_with_current",
    "hip_available",
    "inspect_qwen_hf_directory",
    "kv_bytes_per_token",
    "load_qwen_decode_benchmark_profile",
    "load_qwen_model_manifest",
    "load_torque_artifact",
    "metal_available",
    "packed_words_for_head_dim",
    "quantize_and_pack_rows",
    "quantize_and_pack_rows_dual",
    "run_qwen_decode_runtime_benchmark",
    "run_synthetic_decode_benchmark",
]

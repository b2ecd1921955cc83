"""CPU oracle for the packed rotated KV-cache decode path.

TEST INFRASTRUCTURE ONLY.  This module is a numpy restatement of the
reference algorithm (cbun/torque-mlx) used to check the HIP implementation.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import it, and only as the checker.  The product package
(``torque-mlx_amd/torque_hip``) never imports it and has no CPU fallback.

Every function cites the reference file:line it restates (paths relative to
``src/torque_mlx/`` in the reference).  How each one is pinned:

* ``packed_words_for_head_dim``   -- known-answer table (tests/test_oracle.py).
* ``fwht_last_axis`` / rotation   -- closed-form Sylvester matrix, round trip,
  norm, ``matrix() == apply(I).T``.
* ``rotation_signs_from_seed``    -- the reference's published synthetic
  benchmark output (docs/benchmark-report.md:21,
  max_abs_error_vs_rotated_reference = 0.0800141841 at S=32, D=64, Hkv=2,
  4-bit, seed 0): ``synthetic_benchmark_error`` reproduces it within 1e-6
  with these signs, and misses it by > 1e-4 with one sign flipped or the two
  vectors exchanged.  Shape, values in {-1,+1} and determinism are checked
  too.
* ``synthetic_benchmark_error``   -- the same published figure.
* ``build_gaussian_codebook``     -- golden vectors written by
  ``tests/golden/gen_gaussian_codebooks.py`` from the reference's own
  ``quantization.py``, plus the Max (1960) Lloyd-Max table.
* ``quantize_argmin`` / ``quantize_boundary_count`` -- the reference's KATs
  and their mutual agreement on finite inputs.
* ``pack_indices`` / ``unpack_indices`` -- brute-force bit-by-bit packer,
  round trip, straddle positions.
* ``streaming_attention_decode``  -- textbook softmax attention in float64,
  single-token closed form, empty-sequence zeros.
* ``rms_scales`` / ``quantize_scaled`` / ``dequantize_scaled`` -- the opt-in
  per-vector scale extension, which has NO reference counterpart (the
  reference's codes index one global codebook, quantization.py:120-148):
  pinned by closed forms (constant rows, zero rows), exact invariance of the
  codes under power-of-two scaling of a row, and the Lloyd-Max distortion of
  N(0, 1) that the normalisation is for (reconstruction error of rows with
  widely varying norms).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from math import ceil, sqrt

import numpy as np

SUPPORTED_BIT_WIDTHS = (2, 3, 4)
SUPPORTED_HEAD_DIMS = (64, 128, 256)
WORD_BITS = 32


# ---------------------------------------------------------------- geometry


def packed_words_for_head_dim(head_dim: int, bit_width: int) -> int:
    """quantization.py:76-81 -- ceil(D * b / 32) uint32 words per vector."""
    if bit_width not in SUPPORTED_BIT_WIDTHS:
        raise ValueError(f"Unsupported bit width: {bit_width}")
    if head_dim <= 0:
        raise ValueError("head_dim must be positive")
    return ceil((head_dim * bit_width) / WORD_BITS)


def kv_bytes_per_token(head_dim: int, bit_width: int, kv_heads: int = 1) -> int:
    """quantization.py:84-86 -- packed K+V bytes per token."""
    return packed_words_for_head_dim(head_dim, bit_width) * 4 * kv_heads * 2


def variant_id(bit_width: int, head_dim: int, fused_weights: bool, rotation_mode: str = "hadamard") -> str:
    """layout.py:6-14."""
    return f"b{bit_width}-h{head_dim}-{rotation_mode}-{'fused' if fused_weights else 'unfused'}"


# ---------------------------------------------------------------- rotation


def fwht_last_axis(values: np.ndarray) -> np.ndarray:
    """rotation.py:19-32 -- unnormalised natural-order Walsh-Hadamard transform.

    Butterflies at step 1, 2, 4, ...: (left + right, left - right), float32.
    """
    result = np.array(values, dtype=np.float32, copy=True)
    head_dim = result.shape[-1]
    step = 1
    while step < head_dim:
        blocks = result.reshape(*result.shape[:-1], -1, 2 * step)
        left = blocks[..., :step].copy()
        right = blocks[..., step : 2 * step].copy()
        blocks[..., :step] = left + right
        blocks[..., step : 2 * step] = left - right
        result = blocks.reshape(result.shape)
        step *= 2
    return result


def rotation_signs_from_seed(head_dim: int, seed: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """rotation.py:75-86 -- (signs_left, signs_right), left drawn first."""
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"Unsupported head dimension for rotation: {head_dim}")
    rng = np.random.default_rng(seed)
    left = rng.choice(np.array([-1.0, 1.0], dtype=np.float32), size=head_dim)
    right = rng.choice(np.array([-1.0, 1.0], dtype=np.float32), size=head_dim)
    return left.astype(np.float32), right.astype(np.float32)


def rotation_apply(values: np.ndarray, signs_left: np.ndarray, signs_right: np.ndarray) -> np.ndarray:
    """rotation.py:88-94 -- Pi x = sL * (H (sR * x)) / sqrt(D), float32."""
    array = np.asarray(values, dtype=np.float32)
    head_dim = array.shape[-1]
    rotated = array * np.asarray(signs_right, dtype=np.float32)
    rotated = fwht_last_axis(rotated) / sqrt(head_dim)
    return rotated * np.asarray(signs_left, dtype=np.float32)


def rotation_inverse(values: np.ndarray, signs_left: np.ndarray, signs_right: np.ndarray) -> np.ndarray:
    """rotation.py:96-102 -- Pi^-1 y = sR * (H (sL * y)) / sqrt(D), float32."""
    array = np.asarray(values, dtype=np.float32)
    head_dim = array.shape[-1]
    rotated = array * np.asarray(signs_left, dtype=np.float32)
    rotated = fwht_last_axis(rotated) / sqrt(head_dim)
    return rotated * np.asarray(signs_right, dtype=np.float32)


def rotation_matrix(signs_left: np.ndarray, signs_right: np.ndarray) -> np.ndarray:
    """rotation.py:104-106 -- matrix() = apply(I).T."""
    head_dim = int(np.asarray(signs_left).shape[0])
    return rotation_apply(np.eye(head_dim, dtype=np.float32), signs_left, signs_right).T


# ---------------------------------------------------------------- codebooks


def build_gaussian_codebook(bit_width: int, *, iterations: int = 32, sample_size: int = 200_000, seed: int = 0) -> np.ndarray:
    """quantization.py:89-117 -- Lloyd-Max centroids for N(0,1), float32, sorted."""
    if bit_width not in SUPPORTED_BIT_WIDTHS:
        raise ValueError(f"Unsupported bit width: {bit_width}")
    rng = np.random.default_rng(seed)
    samples = rng.normal(loc=0.0, scale=1.0, size=sample_size).astype(np.float32)
    levels = 1 << bit_width
    quantiles = np.linspace(0.0, 1.0, levels + 2, dtype=np.float32)[1:-1]
    centroids = np.quantile(samples, quantiles).astype(np.float32)
    for _ in range(iterations):
        boundaries = (centroids[:-1] + centroids[1:]) / 2.0
        assignments = np.searchsorted(boundaries, samples, side="right")
        new_centroids = centroids.copy()
        for idx in range(levels):
            cluster = samples[assignments == idx]
            if cluster.size:
                new_centroids[idx] = cluster.mean(dtype=np.float64)
        if np.allclose(new_centroids, centroids):
            centroids = new_centroids
            break
        centroids = new_centroids
    return np.sort(centroids).astype(np.float32)


def uniform_codebook(bit_width: int) -> np.ndarray:
    """benchmarking.py:16-21 -- linspace(-1, 1, 2^b), float32."""
    return np.linspace(-1.0, 1.0, 1 << bit_width, dtype=np.float32)


def codebook_boundaries(centroids: np.ndarray) -> np.ndarray:
    """quantization.py:128-136 -- float32 midpoints (c_i + c_{i+1}) / 2."""
    c = np.asarray(centroids, dtype=np.float32)
    return ((c[:-1] + c[1:]) / 2.0).astype(np.float32)


# ---------------------------------------------------------------- quantize


def quantize_argmin(values: np.ndarray, centroids: np.ndarray) -> np.ndarray:
    """quantization.py:120-125 -- nearest centroid, first index on ties (numpy cache path)."""
    array = np.asarray(values, dtype=np.float32)
    c = np.asarray(centroids, dtype=np.float32)
    distances = np.abs(array.reshape(-1, 1) - c.reshape(1, -1))
    return np.argmin(distances, axis=1).astype(np.uint8).reshape(array.shape)


def quantize_boundary_count(values: np.ndarray, boundaries: np.ndarray) -> np.ndarray:
    """quantization.py:139-148 and mlx_ops.py:264-273 -- code = sum_k [x > bnd_k] (device path)."""
    array = np.asarray(values, dtype=np.float32)
    b = np.asarray(boundaries, dtype=np.float32)
    return np.sum(array[..., None] > b, axis=-1).astype(np.uint8)


def dequantize(indices: np.ndarray, centroids: np.ndarray) -> np.ndarray:
    """quantization.py:151-153."""
    return np.asarray(centroids, dtype=np.float32)[np.asarray(indices)].astype(np.float32)


# ---------------------------------------------------------------- per-vector scales (extension)


def rms_scales(values: np.ndarray) -> np.ndarray:
    """Per-row scale of ``scale_mode="rms"`` (no reference counterpart): float32 sqrt(mean(x^2)) over the
    last axis, 1 for an all-zero row."""
    v = np.asarray(values, dtype=np.float32).astype(np.float64)
    rms = np.sqrt(np.mean(v * v, axis=-1)).astype(np.float32)
    return np.where(rms > 0, rms, np.float32(1.0)).astype(np.float32)


def quantize_scaled(
    values: np.ndarray, boundaries: np.ndarray, scales: np.ndarray | None = None
) -> tuple[np.ndarray, np.ndarray]:
    """Codes of each row divided by its scale (float32 division; the reference's boundary count,
    quantization.py:139-148, applied to x / s) and the scales; ``scales`` defaults to ``rms_scales``."""
    v = np.asarray(values, dtype=np.float32)
    s = rms_scales(v) if scales is None else np.asarray(scales, dtype=np.float32)
    return quantize_boundary_count((v / s[..., None]).astype(np.float32), boundaries), s


def dequantize_scaled(indices: np.ndarray, centroids: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Centroid x per-row scale, float32."""
    return (dequantize(indices, centroids) * np.asarray(scales, dtype=np.float32)[..., None]).astype(np.float32)


# ---------------------------------------------------------------- bit packing


def pack_indices(indices: np.ndarray, bit_width: int) -> np.ndarray:
    """quantization.py:156-173 -- LSB-first bitstream, literal per-code loop."""
    values = np.asarray(indices, dtype=np.uint32).reshape(-1)
    if np.any(values >= (1 << bit_width)):
        raise ValueError(f"Index out of range for {bit_width}-bit packing")
    words = np.zeros(packed_words_for_head_dim(values.size, bit_width), dtype=np.uint32)
    bit_offset = 0
    for value in values:
        value = int(value)
        word_index = bit_offset // WORD_BITS
        shift = bit_offset % WORD_BITS
        words[word_index] |= np.uint32((value << shift) & 0xFFFFFFFF)
        spill = shift + bit_width - WORD_BITS
        if spill > 0:
            words[word_index + 1] |= np.uint32(value >> (bit_width - spill))
        bit_offset += bit_width
    return words


def pack_indices_batched(indices: np.ndarray, bit_width: int) -> np.ndarray:
    """quantization.py:176-201 -- vectorised over leading axes, same bitstream."""
    values = np.asarray(indices, dtype=np.uint32)
    count = values.shape[-1]
    flat = values.reshape(-1, count)
    if np.any(flat >= (1 << bit_width)):
        raise ValueError(f"Index out of range for {bit_width}-bit packing")
    packed = np.zeros((flat.shape[0], packed_words_for_head_dim(count, bit_width)), dtype=np.uint32)
    for idx in range(count):
        bit_offset = idx * bit_width
        word_index = bit_offset // WORD_BITS
        shift = bit_offset % WORD_BITS
        packed[:, word_index] |= flat[:, idx] << np.uint32(shift)
        spill = shift + bit_width - WORD_BITS
        if spill > 0:
            packed[:, word_index + 1] |= flat[:, idx] >> np.uint32(bit_width - spill)
    return packed.reshape(*values.shape[:-1], packed.shape[-1])


def unpack_indices(words: np.ndarray, bit_width: int, count: int) -> np.ndarray:
    """quantization.py:272-290 -- literal per-code loop."""
    packed = np.asarray(words, dtype=np.uint32).reshape(-1)
    mask = (1 << bit_width) - 1
    out = np.zeros(count, dtype=np.uint8)
    bit_offset = 0
    for idx in range(count):
        word_index = bit_offset // WORD_BITS
        shift = bit_offset % WORD_BITS
        value = int(packed[word_index]) >> shift
        spill = shift + bit_width - WORD_BITS
        if spill > 0:
            value |= (int(packed[word_index + 1]) & ((1 << spill) - 1)) << (bit_width - spill)
        out[idx] = value & mask
        bit_offset += bit_width
    return out


def unpack_indices_batched(words: np.ndarray, bit_width: int, count: int) -> np.ndarray:
    """Vectorised unpack over leading axes; the bit-level rule of mlx_ops.py:52-71.

    value = word[w] >> s, OR word[w+1] << (32 - s) when the code straddles.
    """
    packed = np.asarray(words, dtype=np.uint32)
    lead = packed.shape[:-1]
    flat = packed.reshape(-1, packed.shape[-1]).astype(np.uint64)
    offsets = np.arange(count, dtype=np.int64) * bit_width
    widx = offsets // WORD_BITS
    shift = (offsets % WORD_BITS).astype(np.uint64)
    lo = flat[:, widx] >> shift
    straddle = (offsets % WORD_BITS) + bit_width > WORD_BITS
    hi = np.zeros_like(lo)
    if np.any(straddle):
        nxt = np.minimum(widx + 1, flat.shape[1] - 1)
        hi_all = flat[:, nxt] << (np.uint64(WORD_BITS) - shift)
        hi[:, straddle] = hi_all[:, straddle]
    codes = ((lo | hi) & np.uint64((1 << bit_width) - 1)).astype(np.uint8)
    return codes.reshape(*lead, count)


# ---------------------------------------------------------------- attention


def streaming_attention_decode(query: np.ndarray, keys: np.ndarray, values: np.ndarray) -> np.ndarray:
    """reference.py:8-42 -- online-softmax decode for q_len=1, literal loop.

    Small inputs only (pure-Python loop over the sequence).
    """
    query_vec = np.asarray(query, dtype=np.float32)
    key_matrix = np.asarray(keys, dtype=np.float32)
    value_matrix = np.asarray(values, dtype=np.float32)
    if key_matrix.ndim != 2 or value_matrix.ndim != 2:
        raise ValueError("keys and values must be rank-2 [seq_len, head_dim]")
    if key_matrix.shape != value_matrix.shape:
        raise ValueError("keys and values must share the same shape")
    if query_vec.shape != (key_matrix.shape[1],):
        raise ValueError("query must have shape [head_dim]")
    scale = 1.0 / sqrt(query_vec.shape[0])
    m_prev = -np.inf
    l_prev = 0.0
    out = np.zeros_like(query_vec)
    for key_vec, value_vec in zip(key_matrix, value_matrix):
        score = float(np.dot(query_vec, key_vec) * scale)
        m_new = max(m_prev, score)
        l_scale = 0.0 if np.isneginf(m_prev) else float(np.exp(m_prev - m_new))
        p = float(np.exp(score - m_new))
        out *= l_scale
        out += p * value_vec
        l_prev = l_prev * l_scale + p
        m_prev = m_new
    if l_prev == 0.0:
        return out
    return out / l_prev


def attention_decode_dense(query: np.ndarray, keys: np.ndarray, values: np.ndarray) -> np.ndarray:
    """Vectorised float64 softmax attention, batched: q[..., D], K/V[..., S, D] -> [..., D].

    Mathematically the same as ``streaming_attention_decode`` and as the
    split path of mlx_ops.py:571-595 (scores, softmax(scores / sqrt(D)),
    weighted value sum).  Empty sequences give zeros (cache.py:106-107).
    """
    q = np.asarray(query, dtype=np.float64)
    k = np.asarray(keys, dtype=np.float64)
    v = np.asarray(values, dtype=np.float64)
    if k.shape[-2] == 0:
        return np.zeros(q.shape, dtype=np.float32)
    scores = np.einsum("...d,...sd->...s", q, k) / sqrt(q.shape[-1])
    scores -= scores.max(axis=-1, keepdims=True)
    weights = np.exp(scores)
    weights /= weights.sum(axis=-1, keepdims=True)
    return np.einsum("...s,...sd->...d", weights, v).astype(np.float32)


def decode_packed_reference(
    query_rot: np.ndarray,
    k_codes: np.ndarray,
    v_codes: np.ndarray,
    key_centroids: np.ndarray,
    value_centroids: np.ndarray,
    *,
    bit_width: int,
    head_dim: int,
    key_scales: np.ndarray | None = None,
    value_scales: np.ndarray | None = None,
) -> np.ndarray:
    """Packed decode on already-rotated queries: q[B, D], codes[B, S, W] -> out_rot[B, D].

    Restates mlx_ops.py:571-595 (and the single-head K5 at mlx_ops.py:181-253):
    unpack, centroid gather, softmax(q.k / sqrt(D)), weighted value sum.  With
    per-vector scales [B, S] (the extension, see ``rms_scales``) each token is
    centroid x scale.
    """
    kidx = unpack_indices_batched(k_codes, bit_width, head_dim)
    vidx = unpack_indices_batched(v_codes, bit_width, head_dim)
    keys = dequantize(kidx, key_centroids) if key_scales is None else dequantize_scaled(kidx, key_centroids, key_scales)
    values = (
        dequantize(vidx, value_centroids) if value_scales is None else dequantize_scaled(vidx, value_centroids, value_scales)
    )
    return attention_decode_dense(query_rot, keys, values)


# ---------------------------------------------------------------- cache model


@dataclass
class OracleCache:
    """Numpy model of the packed cache (cache.py:35-227, cache_mlx.py:40-302).

    Storage: codes[L, Hkv, S, W] (uint32) per stream.  Supports the
    reference flags rotate_keys_on_append / rotate_values_on_append /
    rotate_queries_on_decode (cache_mlx.py:52-54), fused_weights
    (cache.py:131-134), GQA queries with kv = q // G (cache_mlx.py:706-722)
    and decode-with-current (cache_mlx.py:236-302).  The quantizer is the
    boundary count of the device path (cache_mlx.py:477-521); on finite
    inputs it equals the argmin of the numpy path (cache.py:84-96).
    """

    bit_width: int
    head_dim: int
    num_layers: int
    kv_heads: int
    key_centroids: np.ndarray
    value_centroids: np.ndarray
    signs_left: np.ndarray
    signs_right: np.ndarray
    fused_weights: bool = False
    rotate_keys_on_append: bool = True
    rotate_values_on_append: bool = True
    rotate_queries_on_decode: bool = True
    k_codes: np.ndarray = field(init=False)
    v_codes: np.ndarray = field(init=False)

    def __post_init__(self) -> None:
        w = packed_words_for_head_dim(self.head_dim, self.bit_width)
        self.k_codes = np.zeros((self.num_layers, self.kv_heads, 0, w), dtype=np.uint32)
        self.v_codes = np.zeros_like(self.k_codes)
        self.key_centroids = np.asarray(self.key_centroids, dtype=np.float32)
        self.value_centroids = np.asarray(self.value_centroids, dtype=np.float32)

    @property
    def sequence_length(self) -> int:
        return int(self.k_codes.shape[2])

    def _rot(self, x: np.ndarray) -> np.ndarray:
        return rotation_apply(x, self.signs_left, self.signs_right)

    def encode(self, x: np.ndarray, *, rotate: bool, centroids: np.ndarray) -> np.ndarray:
        """rotate (optional) -> quantize -> pack; x[..., D] -> codes[..., W]."""
        r = self._rot(x) if rotate else np.asarray(x, dtype=np.float32)
        codes = quantize_boundary_count(r, codebook_boundaries(centroids))
        return pack_indices_batched(codes, self.bit_width)

    def append(self, keys: np.ndarray, values: np.ndarray) -> None:
        """keys/values[L, Hkv, S_new, D] (cache.py:78-96, cache_mlx.py:151-171)."""
        kc = self.encode(keys, rotate=self.rotate_keys_on_append, centroids=self.key_centroids)
        vc = self.encode(values, rotate=self.rotate_values_on_append, centroids=self.value_centroids)
        self.k_codes = np.concatenate([self.k_codes, kc], axis=2)
        self.v_codes = np.concatenate([self.v_codes, vc], axis=2)

    def export_dequantized(self) -> tuple[np.ndarray, np.ndarray]:
        """cache.py:189-214."""
        k = dequantize(unpack_indices_batched(self.k_codes, self.bit_width, self.head_dim), self.key_centroids)
        v = dequantize(unpack_indices_batched(self.v_codes, self.bit_width, self.head_dim), self.value_centroids)
        return k, v

    def decode(self, queries: np.ndarray, current: tuple[np.ndarray, np.ndarray] | None = None) -> np.ndarray:
        """queries[L, Hq, D] -> out[L, Hq, D] (cache.py:98-140, cache_mlx.py:173-302)."""
        q = np.asarray(queries, dtype=np.float32)
        hq = q.shape[1]
        group = hq // self.kv_heads
        q_rot = self._rot(q) if self.rotate_queries_on_decode else q
        k, v = self.export_dequantized()
        if current is not None:
            ck, cv = current
            ck_codes = quantize_boundary_count(
                self._rot(ck) if self.rotate_keys_on_append else np.asarray(ck, np.float32),
                codebook_boundaries(self.key_centroids),
            )
            cv_codes = quantize_boundary_count(
                self._rot(cv) if self.rotate_values_on_append else np.asarray(cv, np.float32),
                codebook_boundaries(self.value_centroids),
            )
            k = np.concatenate([k, dequantize(ck_codes, self.key_centroids)[:, :, None, :]], axis=2)
            v = np.concatenate([v, dequantize(cv_codes, self.value_centroids)[:, :, None, :]], axis=2)
        kv_index = np.arange(hq) // group
        out_rot = attention_decode_dense(q_rot, k[:, kv_index], v[:, kv_index])
        if self.fused_weights:
            return out_rot
        return rotation_inverse(out_rot, self.signs_left, self.signs_right)


# ---------------------------------------------------------------- synthetic data


def synthetic_qkv(
    *,
    seed: int,
    num_layers: int,
    kv_heads: int,
    query_heads: int,
    seq_len: int,
    head_dim: int,
    std: float = 1.0,
    outliers: bool = True,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Seeded fp16 Q/K/V as the workload configs describe.

    Q[L, Hq, D], K/V[L, Hkv, S, D] drawn N(0, std) in float32 and cast to
    float16; K gets one log-normal(0, 1) scale per (layer, KV head, channel),
    fixed across tokens (outlier channels).
    """
    rng = np.random.default_rng(seed)
    q = rng.normal(0.0, std, size=(num_layers, query_heads, head_dim)).astype(np.float32)
    k = rng.normal(0.0, std, size=(num_layers, kv_heads, seq_len, head_dim)).astype(np.float32)
    v = rng.normal(0.0, std, size=(num_layers, kv_heads, seq_len, head_dim)).astype(np.float32)
    if outliers:
        k *= rng.lognormal(0.0, 1.0, size=(num_layers, kv_heads, 1, head_dim)).astype(np.float32)
    return q.astype(np.float16), k.astype(np.float16), v.astype(np.float16)


def synthetic_benchmark_error(
    *,
    seq_len: int,
    head_dim: int,
    kv_heads: int,
    bit_width: int,
    seed: int,
    signs: tuple[np.ndarray, np.ndarray] | None = None,
) -> float:
    """benchmarking.py:24-86 -- ``max_abs_error_vs_rotated_reference`` of the synthetic benchmark.

    The numpy cache path of the reference, step for step: N(0, 1) keys
    [S, Hkv, D], values and query [Hkv, D] drawn from ``default_rng(seed)`` in
    that order (benchmarking.py:32-45); Gaussian codebooks with seeds ``seed``
    and ``seed + 1`` and signs ``from_seed(seed)`` (cache.py:47-58); per token
    rotate -> argmin quantize -> pack (cache.py:78-96); decode = rotate the
    query, unpack, dequantize, streaming attention, inverse rotation
    (cache.py:98-140); baseline = streaming attention over the rotated float32
    K/V, rotated back (benchmarking.py:62-71).  ``signs`` overrides the sign
    pair (tests use it to show that the published figure discriminates).
    """
    rng = np.random.default_rng(seed)
    keys = rng.normal(size=(seq_len, kv_heads, head_dim)).astype(np.float32)
    values = rng.normal(size=(seq_len, kv_heads, head_dim)).astype(np.float32)
    query = rng.normal(size=(kv_heads, head_dim)).astype(np.float32)
    kcent = build_gaussian_codebook(bit_width, seed=seed)
    vcent = build_gaussian_codebook(bit_width, seed=seed + 1)
    sl, sr = rotation_signs_from_seed(head_dim, seed) if signs is None else signs
    err = 0.0
    for h in range(kv_heads):
        k_rot = rotation_apply(keys[:, h], sl, sr)
        v_rot = rotation_apply(values[:, h], sl, sr)
        k_words = [pack_indices(quantize_argmin(row, kcent), bit_width) for row in k_rot]
        v_words = [pack_indices(quantize_argmin(row, vcent), bit_width) for row in v_rot]
        k_deq = np.stack([dequantize(unpack_indices(w, bit_width, head_dim), kcent) for w in k_words])
        v_deq = np.stack([dequantize(unpack_indices(w, bit_width, head_dim), vcent) for w in v_words])
        q_rot = rotation_apply(query[h], sl, sr)
        quantized = rotation_inverse(streaming_attention_decode(q_rot, k_deq, v_deq), sl, sr)
        baseline = rotation_inverse(streaming_attention_decode(q_rot, k_rot, v_rot), sl, sr)
        err = max(err, float(np.max(np.abs(quantized - baseline))))
    return err

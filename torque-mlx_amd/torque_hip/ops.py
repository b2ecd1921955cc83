"""Operator API for the packed decode path, mirroring the reference's
``mlx_ops`` wrappers (mlx_ops.py:342-692) with HIP kernels underneath.

Inputs may be numpy arrays or torch tensors; results are float32 / uint32
torch tensors on the current HIP device.  Shapes, argument names and the
``ValueError`` checks follow the reference wrappers.
"""

from __future__ import annotations

from math import sqrt
from typing import Any

import torch

from torque_hip import _lib
from torque_hip._lib import TQ_F32, hip_available
from torque_hip._tensors import codes_to_device, device, dtype_code, shape_of, stream_handle, to_device
from torque_hip.layout import PackedKVLayout

__all__ = [
    "accumulate_packed_values",
    "accumulate_packed_values_batched",
    "decode_packed_attention",
    "decode_packed_attention_split",
    "decode_packed_attention_split_batched",
    "decode_packed_attention_split_batched_with_current",
    "hip_available",
    "metal_available",
    "quantize_and_pack_rows",
    "quantize_and_pack_rows_dual",
    "score_packed_query",
    "score_packed_query_batched",
    "softmax_rows",
    "Workspace",
]

# Reference name of the availability probe (mlx_ops.py:34-45).
metal_available = hip_available


def _as_uint32(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint32)


class Workspace:
    """Split-K workspace, one per (device, stream), grown on demand.

    It holds the per-split partial results between the split kernel and the
    merge kernel of one decode call; every call overwrites what it reads, so
    calls ordered on one stream can share it.
    """

    _pool: dict[tuple[str, int], torch.Tensor] = {}

    @classmethod
    def get(cls, nbytes: int, dev: torch.device) -> torch.Tensor:
        key = (str(dev), stream_handle(dev))
        buf = cls._pool.get(key)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                torch.cuda.current_stream(dev).synchronize()
            buf = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=dev)
            cls._pool[key] = buf
        return buf


def num_cus(dev: torch.device) -> int:
    return int(torch.cuda.get_device_properties(dev).multi_processor_count)


def plan_splits(
    num_layers: int,
    kv_heads: int,
    query_heads: int,
    head_dim: int,
    seq_len: int,
    dev: torch.device,
    *,
    bit_width: int = 0,
    flags: int = 0,
) -> int:
    """The library's default split count for a decode over ``bit_width``-bit rows (0: dense rows)."""
    return _lib.call(
        "tq_decode_default_splits", num_layers, kv_heads, query_heads, head_dim, bit_width, flags, seq_len, num_cus(dev)
    )


def workspace_for(num_layers: int, kv_heads: int, query_heads: int, head_dim: int, n_splits: int, dev: torch.device) -> torch.Tensor:
    nbytes = _lib.call("tq_decode_workspace_bytes", num_layers, kv_heads, query_heads, head_dim, n_splits, num_cus(dev))
    return Workspace.get(int(nbytes), dev)


def packed_decode(
    query: torch.Tensor,
    *,
    num_layers: int,
    query_heads: int,
    kv_heads: int,
    head_dim: int,
    bit_width: int,
    key_codes: torch.Tensor,
    value_codes: torch.Tensor,
    capacity: int,
    seq_len: int,
    key_centroids: torch.Tensor,
    value_centroids: torch.Tensor,
    signs_left: torch.Tensor | None = None,
    signs_right: torch.Tensor | None = None,
    rotate_query: bool = False,
    inverse_output: bool = False,
    current_keys: torch.Tensor | None = None,
    current_values: torch.Tensor | None = None,
    n_splits: int | None = None,
    out: torch.Tensor | None = None,
    key_scales: torch.Tensor | None = None,
    value_scales: torch.Tensor | None = None,
    f32_products: bool = False,
    matrix_products: bool = False,
) -> torch.Tensor:
    """One ``tq_decode`` launch on device tensors; returns out[L, Hq, D] float32.

    With ``key_scales`` / ``value_scales`` ([L, Hkv, capacity] float32, slabs
    written by ``tq_append_scaled``) the launch is ``tq_decode_scaled``.
    ``f32_products`` selects the float32-product split kernel (TQ_F32_PRODUCTS)
    where the float16-split matrix kernel would run; scaled decodes always
    take it (the library adds the flag), so their split plan does too.
    ``matrix_products`` (TQ_MATRIX_PRODUCTS) runs the matrix kernel wherever it
    can, also where the default plan leaves too few rows per split for it.
    """
    dev = query.device
    scaled = key_scales is not None or value_scales is not None
    flags = (_lib.TQ_ROTATE_QUERY if rotate_query else 0) | (_lib.TQ_INVERSE_OUTPUT if inverse_output else 0)
    flags |= _lib.TQ_F32_PRODUCTS if f32_products or scaled else 0
    flags |= _lib.TQ_MATRIX_PRODUCTS if matrix_products else 0
    if n_splits is None or n_splits <= 0:
        n_splits = plan_splits(num_layers, kv_heads, query_heads, head_dim, seq_len, dev, bit_width=bit_width,
                               flags=flags)
    ws = workspace_for(num_layers, kv_heads, query_heads, head_dim, n_splits, dev)
    if out is None:
        out = torch.empty((num_layers, query_heads, head_dim), dtype=torch.float32, device=dev)
    if scaled and (key_scales is None or value_scales is None):
        raise ValueError("key_scales and value_scales must both be given or both be None")
    scale_args = (key_scales.data_ptr(), value_scales.data_ptr()) if scaled else ()
    _lib.call(
        "tq_decode_scaled" if scaled else "tq_decode",
        query.data_ptr(),
        dtype_code(query),
        num_layers,
        query_heads,
        kv_heads,
        head_dim,
        bit_width,
        key_codes.data_ptr(),
        value_codes.data_ptr(),
        *scale_args,
        capacity,
        seq_len,
        key_centroids.data_ptr(),
        value_centroids.data_ptr(),
        None if signs_left is None else signs_left.data_ptr(),
        None if signs_right is None else signs_right.data_ptr(),
        flags,
        None if current_keys is None else current_keys.data_ptr(),
        None if current_values is None else current_values.data_ptr(),
        n_splits,
        ws.data_ptr(),
        ws.numel(),
        out.data_ptr(),
        stream_handle(dev),
    )
    return out


def packed_decode_append(
    query: torch.Tensor,
    new_keys: torch.Tensor,
    new_values: torch.Tensor,
    *,
    num_layers: int,
    query_heads: int,
    kv_heads: int,
    head_dim: int,
    bit_width: int,
    key_codes: torch.Tensor,
    value_codes: torch.Tensor,
    capacity: int,
    seq_len: int,
    key_centroids: torch.Tensor,
    value_centroids: torch.Tensor,
    key_boundaries: torch.Tensor,
    value_boundaries: torch.Tensor,
    signs_left: torch.Tensor,
    signs_right: torch.Tensor,
    rotate_keys: bool = True,
    rotate_values: bool = True,
    rotate_query: bool = False,
    inverse_output: bool = False,
    n_splits: int | None = None,
    out: torch.Tensor | None = None,
    matrix_products: bool = False,
) -> torch.Tensor:
    """One ``tq_decode_append`` launch: pack the new token [L, Hkv, D] into the slabs at row ``seq_len`` and
    decode over the ``seq_len + 1`` tokens.  new_keys and new_values share one dtype (float32 or float16), which
    need not be the query's: the token is quantized from its own values."""
    if new_keys.dtype != new_values.dtype:
        raise ValueError("new_keys and new_values must share one dtype")
    dev = query.device
    append_flags = (_lib.TQ_ROTATE_KEYS if rotate_keys else 0) | (_lib.TQ_ROTATE_VALUES if rotate_values else 0)
    decode_flags = (_lib.TQ_ROTATE_QUERY if rotate_query else 0) | (_lib.TQ_INVERSE_OUTPUT if inverse_output else 0)
    decode_flags |= _lib.TQ_MATRIX_PRODUCTS if matrix_products else 0
    if n_splits is None or n_splits <= 0:
        n_splits = plan_splits(num_layers, kv_heads, query_heads, head_dim, seq_len, dev, bit_width=bit_width,
                               flags=decode_flags)
    ws = workspace_for(num_layers, kv_heads, query_heads, head_dim, n_splits, dev)
    if out is None:
        out = torch.empty((num_layers, query_heads, head_dim), dtype=torch.float32, device=dev)
    _lib.call(
        "tq_decode_append",
        query.data_ptr(),
        dtype_code(query),
        new_keys.data_ptr(),
        new_values.data_ptr(),
        dtype_code(new_keys),
        num_layers,
        query_heads,
        kv_heads,
        head_dim,
        bit_width,
        key_codes.data_ptr(),
        value_codes.data_ptr(),
        capacity,
        seq_len,
        key_centroids.data_ptr(),
        value_centroids.data_ptr(),
        key_boundaries.data_ptr(),
        value_boundaries.data_ptr(),
        signs_left.data_ptr(),
        signs_right.data_ptr(),
        append_flags,
        decode_flags,
        n_splits,
        ws.data_ptr(),
        ws.numel(),
        out.data_ptr(),
        stream_handle(dev),
    )
    return out


def dense_decode(
    query: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    *,
    num_layers: int,
    query_heads: int,
    kv_heads: int,
    head_dim: int,
    capacity: int,
    seq_len: int,
    signs_left: torch.Tensor | None = None,
    signs_right: torch.Tensor | None = None,
    rotate_query: bool = False,
    inverse_output: bool = False,
    n_splits: int | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One ``tq_decode_dense`` launch: dense fp16/fp32 K/V slabs [L, Hkv, capacity, D]."""
    dev = query.device
    if n_splits is None or n_splits <= 0:
        n_splits = plan_splits(num_layers, kv_heads, query_heads, head_dim, seq_len, dev)
    ws = workspace_for(num_layers, kv_heads, query_heads, head_dim, n_splits, dev)
    if out is None:
        out = torch.empty((num_layers, query_heads, head_dim), dtype=torch.float32, device=dev)
    flags = (_lib.TQ_ROTATE_QUERY if rotate_query else 0) | (_lib.TQ_INVERSE_OUTPUT if inverse_output else 0)
    _lib.call(
        "tq_decode_dense",
        query.data_ptr(),
        dtype_code(query),
        keys.data_ptr(),
        values.data_ptr(),
        dtype_code(keys),
        num_layers,
        query_heads,
        kv_heads,
        head_dim,
        capacity,
        seq_len,
        None if signs_left is None else signs_left.data_ptr(),
        None if signs_right is None else signs_right.data_ptr(),
        flags,
        n_splits,
        ws.data_ptr(),
        ws.numel(),
        out.data_ptr(),
        stream_handle(dev),
    )
    return out


# ------------------------------------------------------------------ append / pack


def _check_rows(values_shape: tuple[int, ...], head_dim: int, label: str) -> None:
    if len(values_shape) != 2 or values_shape[1] != head_dim:
        raise ValueError(f"{label} must have shape (rows, {head_dim}), got {values_shape}")


def _check_boundaries(shape: tuple[int, ...], bit_width: int, label: str) -> None:
    expected = (1 << bit_width) - 1
    if len(shape) != 1 or shape[0] != expected:
        raise ValueError(f"{label} must have shape ({expected},), got {shape}")


def quantize_and_pack_rows(values: Any, boundaries: Any, *, bit_width: int, head_dim: int) -> torch.Tensor:
    """values[R, D] (already rotated) -> packed uint32 [R, W] (mlx_ops.py:342-371)."""
    layout = PackedKVLayout(bit_width=bit_width, head_dim=head_dim)
    _check_rows(shape_of(values), head_dim, "values")
    _check_boundaries(shape_of(boundaries), bit_width, "boundaries")
    dev = device()
    x = to_device(values, dev, keep_f16=False)
    bnd = to_device(boundaries, dev, keep_f16=False)
    rows = int(x.shape[0])
    out = torch.empty((rows, layout.packed_words), dtype=torch.int32, device=dev)
    _lib.call(
        "tq_quantize_pack", x.data_ptr(), rows, head_dim, bit_width, bnd.data_ptr(), out.data_ptr(), stream_handle(dev)
    )
    return _as_uint32(out)


def quantize_and_pack_rows_dual(
    values_a: Any, values_b: Any, boundaries_a: Any, boundaries_b: Any, *, bit_width: int, head_dim: int
) -> tuple[torch.Tensor, torch.Tensor]:
    """Two streams with separate boundaries (mlx_ops.py:374-412), one fused launch."""
    layout = PackedKVLayout(bit_width=bit_width, head_dim=head_dim)
    sa, sb = shape_of(values_a), shape_of(values_b)
    _check_rows(sa, head_dim, "values_a")
    if sa != sb:
        raise ValueError(f"values_a and values_b must match, got {sa} and {sb}")
    _check_boundaries(shape_of(boundaries_a), bit_width, "boundaries_a")
    _check_boundaries(shape_of(boundaries_b), bit_width, "boundaries_b")
    dev = device()
    a = to_device(values_a, dev, keep_f16=False)
    b = to_device(values_b, dev, keep_f16=False)
    ba = to_device(boundaries_a, dev, keep_f16=False)
    bb = to_device(boundaries_b, dev, keep_f16=False)
    rows = int(a.shape[0])
    out_a = torch.empty((rows, layout.packed_words), dtype=torch.int32, device=dev)
    out_b = torch.empty_like(out_a)
    _lib.call(
        "tq_append",
        a.data_ptr(),
        b.data_ptr(),
        TQ_F32,
        1,
        1,
        rows,
        head_dim,
        bit_width,
        None,
        None,
        0,
        ba.data_ptr(),
        bb.data_ptr(),
        out_a.data_ptr(),
        out_b.data_ptr(),
        rows,
        0,
        stream_handle(dev),
    )
    return _as_uint32(out_a), _as_uint32(out_b)


# Reference names (mlx_ops.py:342, 374).
quantize_and_pack_rows_metal = quantize_and_pack_rows
quantize_and_pack_rows_dual_metal = quantize_and_pack_rows_dual


# ------------------------------------------------------------------ split path stages


def _packed_batch(packed: Any, layout: PackedKVLayout, dev: torch.device, label: str) -> torch.Tensor:
    shape = shape_of(packed)
    if len(shape) != 3 or shape[2] != layout.packed_words:
        raise ValueError(f"{label} must have shape (batch, seq, {layout.packed_words}), got {shape}")
    return codes_to_device(packed, dev)


def score_packed_query_batched(query: Any, packed: Any, centroids: Any, *, bit_width: int, head_dim: int) -> torch.Tensor:
    """Raw scores q . c[code] over packed rows: [B, D] x [B, S, W] -> [B, S] (mlx_ops.py:501-531)."""
    layout = PackedKVLayout(bit_width=bit_width, head_dim=head_dim)
    qs = shape_of(query)
    if len(qs) != 2 or qs[1] != head_dim:
        raise ValueError(f"batched query must have shape (batch, {head_dim}), got {qs}")
    dev = device()
    codes = _packed_batch(packed, layout, dev, "batched packed codes")
    q = to_device(query, dev, keep_f16=False)
    cent = to_device(centroids, dev, keep_f16=False)
    batch, seq_len = int(codes.shape[0]), int(codes.shape[1])
    scores = torch.empty((batch, seq_len), dtype=torch.float32, device=dev)
    _lib.call(
        "tq_score_packed",
        q.data_ptr(),
        codes.data_ptr(),
        batch,
        seq_len,
        head_dim,
        bit_width,
        cent.data_ptr(),
        scores.data_ptr(),
        stream_handle(dev),
    )
    return scores


def softmax_rows(scores: Any, scale: float) -> torch.Tensor:
    """softmax(scale * scores) over the last axis of [B, S]."""
    dev = device()
    s = to_device(scores, dev, keep_f16=False)
    batch, seq_len = int(s.shape[0]), int(s.shape[1])
    w = torch.empty_like(s)
    _lib.call("tq_softmax_rows", s.data_ptr(), batch, seq_len, float(scale), w.data_ptr(), stream_handle(dev))
    return w


def accumulate_packed_values_batched(
    weights: Any, packed: Any, centroids: Any, *, bit_width: int, head_dim: int
) -> torch.Tensor:
    """sum_t w[b, t] c[code[b, t, :]]: [B, S] x [B, S, W] -> [B, D] (mlx_ops.py:534-568)."""
    layout = PackedKVLayout(bit_width=bit_width, head_dim=head_dim)
    ws = shape_of(weights)
    if len(ws) != 2:
        raise ValueError(f"batched weights must have shape (batch, seq), got {ws}")
    dev = device()
    codes = _packed_batch(packed, layout, dev, "batched packed codes")
    if int(codes.shape[0]) != ws[0] or int(codes.shape[1]) != ws[1]:
        raise ValueError("batched packed codes and weights must agree on batch and sequence dimensions")
    w = to_device(weights, dev, keep_f16=False)
    cent = to_device(centroids, dev, keep_f16=False)
    batch, seq_len = ws
    out = torch.empty((batch, head_dim), dtype=torch.float32, device=dev)
    _lib.call(
        "tq_accumulate_packed",
        w.data_ptr(),
        codes.data_ptr(),
        batch,
        seq_len,
        head_dim,
        bit_width,
        cent.data_ptr(),
        out.data_ptr(),
        stream_handle(dev),
    )
    return out


def _check_width(packed: Any, layout: PackedKVLayout) -> None:
    if shape_of(packed)[-1] != layout.packed_words:
        raise ValueError(f"packed width mismatch: expected {layout.packed_words}, got {shape_of(packed)[-1]}")


def score_packed_query(query: Any, packed: Any, centroids: Any, *, bit_width: int, head_dim: int) -> torch.Tensor:
    """Single-head raw scores [D] x [S, W] -> [S] (mlx_ops.py:415-441)."""
    layout = PackedKVLayout(bit_width=bit_width, head_dim=head_dim)
    _check_width(packed, layout)
    dev = device()
    q = to_device(query, dev, keep_f16=False).reshape(1, head_dim)
    codes = codes_to_device(packed, dev).reshape(1, -1, layout.packed_words)
    return score_packed_query_batched(q, codes, centroids, bit_width=bit_width, head_dim=head_dim)[0]


def accumulate_packed_values(weights: Any, packed: Any, centroids: Any, *, bit_width: int, head_dim: int) -> torch.Tensor:
    """Single-head weighted value sum [S] x [S, W] -> [D] (mlx_ops.py:444-471)."""
    layout = PackedKVLayout(bit_width=bit_width, head_dim=head_dim)
    _check_width(packed, layout)
    dev = device()
    w = to_device(weights, dev, keep_f16=False).reshape(1, -1)
    codes = codes_to_device(packed, dev).reshape(1, -1, layout.packed_words)
    return accumulate_packed_values_batched(w, codes, centroids, bit_width=bit_width, head_dim=head_dim)[0]


def decode_packed_attention_split(
    query: Any, k_codes: Any, v_codes: Any, centroids_k: Any, centroids_v: Any, *, bit_width: int, head_dim: int
) -> torch.Tensor:
    """Three-stage decode (score, softmax, values) for one head (mlx_ops.py:474-498)."""
    scores = score_packed_query(query, k_codes, centroids_k, bit_width=bit_width, head_dim=head_dim)
    weights = softmax_rows(scores.reshape(1, -1), 1.0 / sqrt(head_dim))
    return accumulate_packed_values(weights[0], v_codes, centroids_v, bit_width=bit_width, head_dim=head_dim)


# ------------------------------------------------------------------ fused decode


def _fused_batched(
    query: Any,
    k_codes: Any,
    v_codes: Any,
    centroids_k: Any,
    centroids_v: Any,
    *,
    bit_width: int,
    head_dim: int,
    current_keys: Any = None,
    current_values: Any = None,
    n_splits: int | None = None,
) -> torch.Tensor:
    layout = PackedKVLayout(bit_width=bit_width, head_dim=head_dim)
    dev = device()
    q = to_device(query, dev)
    kc = _packed_batch(k_codes, layout, dev, "packed codes")
    vc = _packed_batch(v_codes, layout, dev, "packed codes")
    batch, seq_len = int(kc.shape[0]), int(kc.shape[1])
    ck = cv = None
    if current_keys is not None:
        ck = to_device(current_keys, dev, keep_f16=False)
        cv = to_device(current_values, dev, keep_f16=False)
    out = packed_decode(
        q,
        num_layers=1,
        query_heads=batch,
        kv_heads=batch,
        head_dim=head_dim,
        bit_width=bit_width,
        key_codes=kc,
        value_codes=vc,
        capacity=seq_len,
        seq_len=seq_len,
        key_centroids=to_device(centroids_k, dev, keep_f16=False),
        value_centroids=to_device(centroids_v, dev, keep_f16=False),
        current_keys=ck,
        current_values=cv,
        n_splits=n_splits,
    )
    return out[0]


def decode_packed_attention_split_batched(
    query: Any, k_codes: Any, v_codes: Any, centroids_k: Any, centroids_v: Any, *, bit_width: int, head_dim: int
) -> torch.Tensor:
    """[B, D] x [B, S, W] -> [B, D]: the ``split_batched`` strategy (mlx_ops.py:571-595).

    One split-K launch with an in-kernel online softmax and log-sum-exp merge
    replaces the reference's score kernel, ``mx.softmax`` and value kernel.
    """
    qs = shape_of(query)
    if len(qs) != 2 or qs[1] != head_dim:
        raise ValueError(f"batched query must have shape (batch, {head_dim}), got {qs}")
    if shape_of(k_codes) != shape_of(v_codes):
        raise ValueError(f"k_codes and v_codes must match, got {shape_of(k_codes)} and {shape_of(v_codes)}")
    if len(shape_of(k_codes)) == 3 and shape_of(k_codes)[0] != qs[0]:
        raise ValueError("packed codes and query must agree on batch dimension")
    return _fused_batched(query, k_codes, v_codes, centroids_k, centroids_v, bit_width=bit_width, head_dim=head_dim)


def decode_packed_attention_split_batched_with_current(
    query: Any,
    k_codes: Any,
    v_codes: Any,
    centroids_k: Any,
    centroids_v: Any,
    current_keys: Any,
    current_values: Any,
    *,
    bit_width: int,
    head_dim: int,
) -> torch.Tensor:
    """Packed tokens plus one dense current token per row (mlx_ops.py:598-660)."""
    qs = shape_of(query)
    if len(qs) != 2 or qs[1] != head_dim:
        raise ValueError(f"batched query must have shape (batch, {head_dim}), got {qs}")
    if shape_of(current_keys) != qs:
        raise ValueError(f"current_keys must have shape {qs}, got {shape_of(current_keys)}")
    if shape_of(current_values) != qs:
        raise ValueError(f"current_values must have shape {qs}, got {shape_of(current_values)}")
    if len(shape_of(k_codes)) != 3 or len(shape_of(v_codes)) != 3:
        raise ValueError("packed codes must have shape (batch, seq, packed_words)")
    if shape_of(k_codes) != shape_of(v_codes):
        raise ValueError(f"k_codes and v_codes must match, got {shape_of(k_codes)} and {shape_of(v_codes)}")
    if shape_of(k_codes)[0] != qs[0]:
        raise ValueError("packed codes and query must agree on batch dimension")
    return _fused_batched(
        query,
        k_codes,
        v_codes,
        centroids_k,
        centroids_v,
        bit_width=bit_width,
        head_dim=head_dim,
        current_keys=current_keys,
        current_values=current_values,
    )


def decode_packed_attention(
    query: Any, k_codes: Any, v_codes: Any, centroids_k: Any, centroids_v: Any, *, bit_width: int, head_dim: int
) -> torch.Tensor:
    """Single-head fused decode [D] x [S, W] -> [D] (mlx_ops.py:663-692)."""
    layout = PackedKVLayout(bit_width=bit_width, head_dim=head_dim)
    if shape_of(k_codes)[-1] != layout.packed_words or shape_of(v_codes)[-1] != layout.packed_words:
        raise ValueError("packed width mismatch for fused decode kernel")
    dev = device()
    q = to_device(query, dev).reshape(1, head_dim)
    kc = codes_to_device(k_codes, dev).reshape(1, -1, layout.packed_words)
    vc = codes_to_device(v_codes, dev).reshape(1, -1, layout.packed_words)
    return _fused_batched(q, kc, vc, centroids_k, centroids_v, bit_width=bit_width, head_dim=head_dim)[0]

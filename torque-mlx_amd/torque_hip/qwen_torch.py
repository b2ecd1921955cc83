"""PyTorch attention adapter for Qwen-style gated full-attention layers.

The reference patches each full-attention layer of an MLX Qwen model with an
adapter (qwen_mlx.py:766-864, ``vo_only_runtime_qk_rotation``): query / gate,
key and value projections, per-head RMS norms on queries and keys, rotary
embeddings; a multi-token chunk runs dense attention over a dense cache and
appends the chunk to the packed cache; a one-token step decodes through the
packed cache with the current token and then appends it; the result, which is
in the rotated basis, is rotated back, gated by ``sigmoid(gate)`` and sent
through the output projection.  Values come out of a value projection whose
head blocks were pre-multiplied by the rotation (families/qwen.py:439-453,
473-557), so the cache stores them as they are; queries and keys are rotated
at run time (qwen_mlx.py:736-763: rotate keys on append, queries on decode,
not values).

Here the same adapter wraps a ``torch.nn.Module`` shaped like transformers'
``Qwen3NextAttention`` (``q_proj`` giving (query, gate) per head, ``k_proj``,
``v_proj``, ``o_proj``, ``q_norm``, ``k_norm``; rotary ``(cos, sin)`` passed to
``forward``), and the cache is a ``TorqueKVCacheHIP``.  The one-token step is a
single ``tq_decode_append`` launch (decode with the current token, then
append, fused).  The reference loads pre-fused weights from its artifact and
restores the output projection at run time (qwen_mlx.py:610-618, 773-779);
starting from a model's own weights, ``patch_vo_only_qwen_attention`` instead
rotates the value projection and keeps the output projection — the weights the
adapter runs with are the same.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Callable

import numpy as np
import torch
import torch.nn.functional as F

from torque_hip.cache_hip import TorqueKVCacheHIP
from torque_hip.config import TorqueConfig
from torque_hip.quantization import Codebook
from torque_hip.rotation import RotationSpec

DEFAULT_QWEN_DECODE_TAIL_CAPACITY = 64


# ---------------------------------------------------------------- weight helpers


def _rotation_matrix(rotation: RotationSpec, dev: torch.device) -> torch.Tensor:
    return torch.as_tensor(rotation.matrix(), dtype=torch.float32, device=dev)


def rotate_stacked_output_projection(
    weight: torch.Tensor, *, head_dim: int, num_blocks: int, rotation: RotationSpec
) -> torch.Tensor:
    """Each head block of an output projection times the rotation: W_b -> Pi W_b (families/qwen.py:439-453).

    ``weight`` is [num_blocks * head_dim, in] (a bias is a [num_blocks * head_dim] vector); float32 result.
    """
    w = weight.detach().to(torch.float32)
    if w.shape[0] != num_blocks * head_dim:
        raise ValueError(f"Expected projection output dim {num_blocks * head_dim}, got {w.shape[0]}")
    rot = _rotation_matrix(rotation, w.device)
    blocks = w.reshape(num_blocks, head_dim, -1)
    return torch.matmul(rot[None], blocks).reshape(w.shape)


def inverse_rotate_stacked_input_projection(
    weight: torch.Tensor, *, head_dim: int, num_blocks: int, rotation: RotationSpec
) -> torch.Tensor:
    """Each head block of an input projection times the inverse rotation: W_b -> W_b Pi^T (families/qwen.py:456-470)."""
    w = weight.detach().to(torch.float32)
    if w.shape[1] != num_blocks * head_dim:
        raise ValueError(f"Expected projection input dim {num_blocks * head_dim}, got {w.shape[1]}")
    rot = _rotation_matrix(rotation, w.device)
    return torch.matmul(w.reshape(w.shape[0], num_blocks, head_dim), rot.T).reshape(w.shape)


def restore_stacked_input_projection(
    weight: torch.Tensor, *, head_dim: int, num_blocks: int, rotation: RotationSpec
) -> torch.Tensor:
    """Undo ``inverse_rotate_stacked_input_projection``: W_b -> W_b Pi (qwen_mlx.py:610-618)."""
    w = weight.detach().to(torch.float32)
    if w.shape[1] != num_blocks * head_dim:
        raise ValueError(f"Expected projection input dim {num_blocks * head_dim}, got {w.shape[1]}")
    rot = _rotation_matrix(rotation, w.device)
    return torch.matmul(w.reshape(w.shape[0], num_blocks, head_dim), rot).reshape(w.shape)


def runtime_unrotate_attention_output(attn_output: torch.Tensor, *, rotation: RotationSpec) -> torch.Tensor:
    """Inverse rotation of every head row of an attention output (qwen_mlx.py:621-630); float32 result."""
    if int(attn_output.shape[-1]) != rotation.head_dim:
        raise ValueError(f"Expected last dimension {rotation.head_dim}, got {int(attn_output.shape[-1])}")
    return rotation.inverse_device(attn_output.contiguous()).reshape(attn_output.shape)


# ---------------------------------------------------------------- per-layer cache


@dataclass
class QwenTorqueFullAttentionCacheHIP:
    """Per-layer cache of the adapter (qwen_mlx.py:633-734): a packed ``TorqueKVCacheHIP`` plus the
    dense keys / values of the prompt chunks, which only multi-token chunks attend to."""

    torque_cache: TorqueKVCacheHIP
    dense_keys: torch.Tensor | None = field(default=None)
    dense_values: torch.Tensor | None = field(default=None)
    decode_mode: bool = field(default=False)

    @property
    def offset(self) -> int:
        return self.torque_cache.offset

    @property
    def state(self) -> list[torch.Tensor]:
        state = [self.torque_cache._key_codes, self.torque_cache._value_codes]
        if self.dense_keys is not None:
            state.extend([self.dense_keys, self.dense_values])
        return state

    def make_mask(self, N: int, *, window_size: int | None = None, return_array: bool = False) -> Any:
        return self.torque_cache.make_mask(N, window_size=window_size, return_array=return_array)

    def update_dense_and_fetch(self, keys: torch.Tensor, values: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Append a chunk's [1, Hkv, L, D] keys / values to the dense cache and return all of it."""
        if self.decode_mode:
            if self.offset > 0:
                raise RuntimeError("Torque HIP cache cannot process a multi-token chunk after switching to decode mode")
            self.decode_mode = False
        if self.dense_keys is None:
            self.dense_keys, self.dense_values = keys, values
        else:
            self.dense_keys = torch.cat([self.dense_keys, keys], dim=2)
            self.dense_values = torch.cat([self.dense_values, values], dim=2)
        return self.dense_keys, self.dense_values

    def _append_tokens(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        if int(keys.shape[0]) != 1:
            raise ValueError("Torque HIP Qwen cache currently supports batch size 1")
        self.torque_cache.append_many(key=keys[0], value=values[0])

    def append_prompt_tokens(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        self._append_tokens(keys, values)

    def append_decode_tokens(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        self._append_tokens(keys, values)

    def _enter_decode(self, queries: torch.Tensor) -> None:
        if int(queries.shape[0]) != 1 or int(queries.shape[2]) != 1:
            raise ValueError("Torque HIP Qwen decode currently supports batch size 1 and q_len=1")
        self.decode_mode = True
        self.dense_keys = self.dense_values = None

    @staticmethod
    def _check_current(keys: torch.Tensor, values: torch.Tensor) -> None:
        if int(keys.shape[0]) != 1 or int(keys.shape[2]) != 1 or int(values.shape[0]) != 1 or int(values.shape[2]) != 1:
            raise ValueError("Torque HIP Qwen decode currently expects single-token key/value updates")

    def decode_token(self, queries: torch.Tensor) -> torch.Tensor:
        """[1, Hq, 1, D] queries -> [1, Hq, 1, D] output over the packed cache (qwen_mlx.py:692-708)."""
        self._enter_decode(queries)
        out = self.torque_cache.decode(query=queries[0, :, 0, :], return_numpy=False)
        return out.reshape(1, int(queries.shape[1]), 1, int(queries.shape[3]))

    def decode_token_with_current(self, queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor) -> torch.Tensor:
        """Decode with the current token, cache unchanged (qwen_mlx.py:710-733)."""
        self._enter_decode(queries)
        self._check_current(keys, values)
        out = self.torque_cache.decode_with_current(query=queries[0, :, 0, :], key=keys[0], value=values[0],
                                                    return_numpy=False)
        return out.reshape(1, int(queries.shape[1]), 1, int(queries.shape[3]))

    def decode_token_and_append(self, queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor) -> torch.Tensor:
        """``decode_token_with_current`` then ``append_decode_tokens`` of the same token, in one launch."""
        self._enter_decode(queries)
        self._check_current(keys, values)
        out = self.torque_cache.decode_append(query=queries[0, :, 0, :], key=keys[0], value=values[0],
                                              return_numpy=False)
        return out.reshape(1, int(queries.shape[1]), 1, int(queries.shape[3]))


def build_qwen_torque_cache(
    *,
    bit_width: int,
    head_dim: int,
    kv_heads: int,
    rotation_seed: int = 0,
    rotation_mode: str = "hadamard",
    key_codebook: Codebook | None = None,
    value_codebook: Codebook | None = None,
    decode_tail_capacity: int = DEFAULT_QWEN_DECODE_TAIL_CAPACITY,
    initial_capacity: int = 256,
) -> QwenTorqueFullAttentionCacheHIP:
    """One layer's cache with the reference's Qwen settings (qwen_mlx.py:736-763): fused weights, keys
    rotated on append, values not (the value projection is pre-rotated), queries rotated on decode."""
    config = TorqueConfig(
        bit_width=bit_width,
        head_dim=head_dim,
        num_layers=1,
        kv_heads=kv_heads,
        fused_weights=True,
        rotation_mode=rotation_mode,
        rotation_seed=rotation_seed,
    )
    return QwenTorqueFullAttentionCacheHIP(
        torque_cache=TorqueKVCacheHIP(
            config=config,
            key_codebook=key_codebook,
            value_codebook=value_codebook,
            initial_capacity=initial_capacity,
            decode_tail_capacity=decode_tail_capacity,
            rotate_keys_on_append=True,
            rotate_values_on_append=False,
            rotate_queries_on_decode=True,
        )
    )


# ---------------------------------------------------------------- attention adapter


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rotary(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotary embedding on the first ``cos.shape[-1]`` dims of [B, H, L, D] queries and keys (rotate-half
    convention, the rest passed through), ``cos`` / ``sin`` of shape [B, L, rotary_dim]."""
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    r = int(cos.shape[-1])
    q_rot, q_pass = q[..., :r], q[..., r:]
    k_rot, k_pass = k[..., :r], k[..., r:]
    q_out = torch.cat([q_rot * cos + _rotate_half(q_rot) * sin, q_pass], dim=-1)
    k_out = torch.cat([k_rot * cos + _rotate_half(k_rot) * sin, k_pass], dim=-1)
    return q_out, k_out


def _dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float, offset: int) -> torch.Tensor:
    """Causal attention of L new queries at positions offset.. over all S cached keys, float32 math."""
    group = int(q.shape[1]) // int(k.shape[1])
    k = k.to(torch.float32).repeat_interleave(group, dim=1)
    v = v.to(torch.float32).repeat_interleave(group, dim=1)
    L, S = int(q.shape[2]), int(k.shape[2])
    rows = torch.arange(offset, offset + L, device=q.device)[:, None]
    cols = torch.arange(S, device=q.device)[None, :]
    return F.scaled_dot_product_attention(q.to(torch.float32), k, v, attn_mask=cols <= rows, scale=scale)


def _check_same_rotation(cache: QwenTorqueFullAttentionCacheHIP, rotation: RotationSpec) -> None:
    # The cache rotates keys and queries with its own signs; the adapter rotates the output back (and the
    # value projection was rotated) with ``rotation``: both must be the same transform.
    own = cache.torque_cache.rotation
    if not (np.array_equal(own.signs_left, rotation.signs_left) and np.array_equal(own.signs_right, rotation.signs_right)):
        raise ValueError("the cache's rotation differs from the adapter's rotation")


class TorqueQwenAttention(torch.nn.Module):
    """Drop-in for a ``Qwen3NextAttention``-style module whose decode runs through the packed cache
    (the reference's ``_TorqueAttentionAdapter``, qwen_mlx.py:788-864).

    ``forward(hidden_states, position_embeddings, attention_mask=None, past_key_values=None)`` returns
    ``(output, None)`` like the wrapped module.  The cache is ``past_key_values`` when that is a
    ``QwenTorqueFullAttentionCacheHIP``, else ``self.cache``; with no cache it is plain dense attention.
    """

    def __init__(self, base_attn: torch.nn.Module, *, rotation: RotationSpec,
                 cache: QwenTorqueFullAttentionCacheHIP | None = None,
                 rotary: Callable[..., tuple[torch.Tensor, torch.Tensor]] = apply_rotary) -> None:
        super().__init__()
        self.base_attn = base_attn
        self.rotation = rotation
        self.cache = cache
        self.rotary = rotary
        self.head_dim = int(getattr(base_attn, "head_dim"))
        if self.head_dim != rotation.head_dim:
            raise ValueError(f"rotation head_dim {rotation.head_dim} does not match the attention's {self.head_dim}")
        if cache is not None:
            _check_same_rotation(cache, rotation)
        self.scaling = float(getattr(base_attn, "scaling", self.head_dim**-0.5))

    def forward(self, hidden_states: torch.Tensor, position_embeddings: tuple[torch.Tensor, torch.Tensor],
                attention_mask: Any = None, past_key_values: Any = None, **kwargs: Any) -> tuple[torch.Tensor, None]:
        attn = self.base_attn
        B, L, _ = hidden_states.shape
        if B != 1:
            raise ValueError("Torque HIP Qwen runtime currently supports batch size 1")
        hd = self.head_dim
        queries, gate = torch.chunk(attn.q_proj(hidden_states).view(B, L, -1, hd * 2), 2, dim=-1)
        gate = gate.reshape(B, L, -1)
        queries = attn.q_norm(queries).transpose(1, 2)
        keys = attn.k_norm(attn.k_proj(hidden_states).view(B, L, -1, hd)).transpose(1, 2)
        values = attn.v_proj(hidden_states).view(B, L, -1, hd).transpose(1, 2)
        cos, sin = position_embeddings
        queries, keys = self.rotary(queries, keys, cos, sin)

        cache = self.cache
        if isinstance(past_key_values, QwenTorqueFullAttentionCacheHIP):
            cache = past_key_values
            _check_same_rotation(cache, self.rotation)
        if cache is not None and L == 1:
            output = cache.decode_token_and_append(queries.float(), keys.float(), values.float())
        elif cache is not None:
            offset = cache.offset
            dense_keys, dense_values = cache.update_dense_and_fetch(keys, values)
            output = _dense_attention(queries, dense_keys, dense_values, scale=self.scaling, offset=offset)
            cache.append_prompt_tokens(keys.float(), values.float())
        else:
            output = _dense_attention(queries, keys, values, scale=self.scaling, offset=0)

        output = runtime_unrotate_attention_output(output, rotation=self.rotation)
        output = output.transpose(1, 2).reshape(B, L, -1)
        projected = (output * torch.sigmoid(gate.float())).to(attn.o_proj.weight.dtype)
        return attn.o_proj(projected), None


@torch.no_grad()
def patch_vo_only_qwen_attention(layer: torch.nn.Module, *, rotation: RotationSpec,
                                 cache: QwenTorqueFullAttentionCacheHIP | None = None) -> TorqueQwenAttention:
    """Replace ``layer.self_attn`` (a module with the reference model's original weights) by the adapter.

    The value projection's head blocks (weight and bias) are multiplied by the rotation in place, as the
    reference's conversion does (families/qwen.py:505-510); the output projection keeps its weights, as
    the reference's run time restores them (qwen_mlx.py:773-779), and the adapter rotates the attention
    output back before the gate.  Returns the adapter.
    """
    attn = layer.self_attn
    hd = int(attn.head_dim)
    v = attn.v_proj
    kv_heads = int(v.weight.shape[0]) // hd
    v.weight.copy_(rotate_stacked_output_projection(v.weight, head_dim=hd, num_blocks=kv_heads, rotation=rotation)
                   .to(v.weight.dtype))
    if v.bias is not None:
        fused_bias = rotate_stacked_output_projection(v.bias[:, None], head_dim=hd, num_blocks=kv_heads, rotation=rotation)
        v.bias.copy_(fused_bias[:, 0].to(v.bias.dtype))
    adapter = TorqueQwenAttention(attn, rotation=rotation, cache=cache)
    layer.self_attn = adapter
    return adapter

"""Qwen-style attention adapter (qwen_mlx.py:766-864) around the packed HIP cache.

* the weight helpers against the oracle's rotation matrix (families/qwen.py:439-470, qwen_mlx.py:610-618);
* a prompt chunk through the patched layer against transformers' own ``Qwen3NextAttention`` with the
  original weights (dense path: fusing V and rotating the output back must cancel exactly);
* decode steps against the oracle pipeline: the same projections, the oracle's packed cache with the
  reference's Qwen flags (keys rotated on append, values pre-rotated, queries rotated, output left
  rotated), its inverse rotation, the gate and the output projection; packed codes bit-exact.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from oracle import torque_oracle as o

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")
from transformers.models.qwen3_next import modeling_qwen3_next as hf  # noqa: E402
from transformers.models.qwen3_next.configuration_qwen3_next import Qwen3NextConfig  # noqa: E402


def _layer(head_dim: int, q_heads: int, kv_heads: int, seed: int):
    cfg = Qwen3NextConfig(hidden_size=q_heads * head_dim, num_attention_heads=q_heads, num_key_value_heads=kv_heads,
                          head_dim=head_dim, partial_rotary_factor=0.25, rms_norm_eps=1e-6, num_hidden_layers=1,
                          vocab_size=32, intermediate_size=64)
    cfg._attn_implementation = "eager"
    torch.manual_seed(seed)
    attn = hf.Qwen3NextAttention(cfg, 0)
    with torch.no_grad():
        attn.q_norm.weight.normal_(0.0, 0.2)
        attn.k_norm.weight.normal_(0.0, 0.2)
    layer = torch.nn.Module()
    layer.self_attn = attn
    return cfg, layer, hf.Qwen3NextRotaryEmbedding(cfg)


def _causal_mask(L: int, offset: int) -> torch.Tensor:
    rows = torch.arange(offset, offset + L)[:, None]
    cols = torch.arange(offset + L)[None, :]
    return torch.where(cols <= rows, 0.0, float("-inf"))[None, None]


def test_projection_helpers_match_oracle_rotation(hip_device):
    from torque_hip import RotationSpec
    from torque_hip import qwen_torch as qt

    rot = RotationSpec.from_seed(head_dim=128, seed=3)
    r = o.rotation_matrix(rot.signs_left, rot.signs_right)
    g = torch.Generator().manual_seed(0)
    w_out = torch.randn(3 * 128, 40, generator=g)
    got = qt.rotate_stacked_output_projection(w_out.to(hip_device), head_dim=128, num_blocks=3, rotation=rot).cpu().numpy()
    exp = np.concatenate([r @ b for b in w_out.numpy().reshape(3, 128, 40)], axis=0)
    np.testing.assert_allclose(got, exp, atol=1e-5, rtol=1e-5)
    w_in = torch.randn(24, 2 * 128, generator=g)
    inv = qt.inverse_rotate_stacked_input_projection(w_in.to(hip_device), head_dim=128, num_blocks=2, rotation=rot)
    exp_inv = (w_in.numpy().reshape(24, 2, 128) @ r.T).reshape(24, 256)
    np.testing.assert_allclose(inv.cpu().numpy(), exp_inv, atol=1e-5, rtol=1e-5)
    back = qt.restore_stacked_input_projection(inv, head_dim=128, num_blocks=2, rotation=rot)
    np.testing.assert_allclose(back.cpu().numpy(), w_in.numpy(), atol=1e-5, rtol=1e-5)
    y = torch.randn(2, 5, 128, generator=g).to(hip_device)
    un = qt.runtime_unrotate_attention_output(y, rotation=rot).cpu().numpy()
    np.testing.assert_allclose(un, o.rotation_inverse(y.cpu().numpy(), rot.signs_left, rot.signs_right), atol=1e-6)
    with pytest.raises(ValueError, match="Expected projection output dim 384, got 40"):
        qt.rotate_stacked_output_projection(w_out.T.to(hip_device), head_dim=128, num_blocks=3, rotation=rot)
    with pytest.raises(ValueError, match="Expected projection input dim 256, got 24"):
        qt.inverse_rotate_stacked_input_projection(w_in.T.to(hip_device), head_dim=128, num_blocks=2, rotation=rot)


@pytest.mark.parametrize("head_dim,q_heads,kv_heads", [(64, 4, 2), (128, 8, 2), (256, 4, 1)])
def test_prompt_chunk_matches_transformers_attention(hip_device, head_dim, q_heads, kv_heads):
    from torque_hip import qwen_torch as qt

    cfg, layer, rope = _layer(head_dim, q_heads, kv_heads, seed=head_dim)
    base = copy.deepcopy(layer.self_attn).to(hip_device)
    layer = layer.to(hip_device)
    cache = qt.build_qwen_torque_cache(bit_width=4, head_dim=head_dim, kv_heads=kv_heads, rotation_seed=5)
    adapter = qt.patch_vo_only_qwen_attention(layer, rotation=cache.torque_cache.rotation, cache=cache)
    g = torch.Generator(device=hip_device).manual_seed(1)
    offset = 0
    for L in (9, 4):  # two prompt chunks: the second attends to the first through the dense cache
        x = torch.randn(1, L, cfg.hidden_size, generator=g, device=hip_device)
        pos = torch.arange(offset, offset + L, device=hip_device)[None]
        cos, sin = rope(x, pos)
        with torch.no_grad():
            got, _ = adapter(x, (cos, sin))
            # transformers' module over the full prefix (it keeps no cache here): recompute all positions
            if offset == 0:
                prefix = x
            else:
                prefix = torch.cat([prev, x], dim=1)
            pcos, psin = rope(prefix, torch.arange(offset + L, device=hip_device)[None])
            exp, _ = base(prefix, (pcos, psin), _causal_mask(offset + L, 0).to(hip_device))
        np.testing.assert_allclose(got.cpu().numpy(), exp[:, offset:].cpu().numpy(), atol=2e-5, rtol=1e-4)
        prev = x if offset == 0 else torch.cat([prev, x], dim=1)
        offset += L
    assert cache.offset == offset == cache.torque_cache.sequence_length


def _qkv(adapter, x, cos, sin):
    from torque_hip import qwen_torch as qt

    attn = adapter.base_attn
    hd = adapter.head_dim
    q, gate = torch.chunk(attn.q_proj(x).view(1, x.shape[1], -1, hd * 2), 2, dim=-1)
    q = attn.q_norm(q).transpose(1, 2)
    k = attn.k_norm(attn.k_proj(x).view(1, x.shape[1], -1, hd)).transpose(1, 2)
    v = attn.v_proj(x).view(1, x.shape[1], -1, hd).transpose(1, 2)
    q, k = qt.apply_rotary(q, k, cos, sin)
    return q, gate.reshape(1, x.shape[1], -1), k, v


@pytest.mark.parametrize("bits,head_dim,q_heads,kv_heads,prompt", [(4, 128, 8, 2, 40), (3, 64, 4, 1, 33), (2, 256, 4, 2, 7)])
def test_decode_steps_match_oracle_pipeline(hip_device, bits, head_dim, q_heads, kv_heads, prompt):
    from torque_hip import qwen_torch as qt

    cfg, layer, rope = _layer(head_dim, q_heads, kv_heads, seed=bits + head_dim)
    layer = layer.to(hip_device)
    cache = qt.build_qwen_torque_cache(bit_width=bits, head_dim=head_dim, kv_heads=kv_heads, rotation_seed=7,
                                       initial_capacity=16)
    rotation = cache.torque_cache.rotation
    adapter = qt.patch_vo_only_qwen_attention(layer, rotation=rotation, cache=cache)
    tc = cache.torque_cache
    model = o.OracleCache(bit_width=bits, head_dim=head_dim, num_layers=1, kv_heads=kv_heads,
                          key_centroids=tc.key_codebook.centroids, value_centroids=tc.value_codebook.centroids,
                          signs_left=rotation.signs_left, signs_right=rotation.signs_right, fused_weights=True,
                          rotate_keys_on_append=True, rotate_values_on_append=False, rotate_queries_on_decode=True)
    g = torch.Generator(device=hip_device).manual_seed(bits)
    x = torch.randn(1, prompt, cfg.hidden_size, generator=g, device=hip_device)
    cos, sin = rope(x, torch.arange(prompt, device=hip_device)[None])
    with torch.no_grad():
        adapter(x, (cos, sin))
        _, _, k, v = _qkv(adapter, x, cos, sin)
    model.append(k[0][None].float().cpu().numpy(), v[0][None].float().cpu().numpy())
    w_o = layer.self_attn.base_attn.o_proj.weight.detach().cpu().numpy().astype(np.float64)
    for step in range(4):
        pos = prompt + step
        x = torch.randn(1, 1, cfg.hidden_size, generator=g, device=hip_device)
        cos, sin = rope(x, torch.tensor([[pos]], device=hip_device))
        with torch.no_grad():
            got, _ = adapter(x, (cos, sin))
            q, gate, k, v = _qkv(adapter, x, cos, sin)
        kk, vv = k[0, :, 0].float().cpu().numpy(), v[0, :, 0].float().cpu().numpy()
        out_rot = model.decode(q[0, :, 0].float().cpu().numpy()[None], current=(kk[None], vv[None]))[0]
        model.append(kk[None, :, None], vv[None, :, None])
        attn_out = o.rotation_inverse(out_rot, rotation.signs_left, rotation.signs_right).reshape(-1)
        gated = attn_out.astype(np.float64) / (1.0 + np.exp(-gate[0, 0].double().cpu().numpy()))
        exp = gated @ w_o.T
        got_np = got[0, 0].double().cpu().numpy()
        err = np.max(np.abs(got_np - exp))
        rel = np.linalg.norm(got_np - exp) / np.linalg.norm(exp)
        assert err <= 2e-3 and rel <= 1e-3, (step, err, rel)
        assert tc.sequence_length == pos + 1
        s = tc.sequence_length
        np.testing.assert_array_equal(tc._key_codes[:, :, :s].cpu().numpy().view(np.uint32), model.k_codes)
        np.testing.assert_array_equal(tc._value_codes[:, :, :s].cpu().numpy().view(np.uint32), model.v_codes)


def test_adapter_cache_errors(hip_device):
    from torque_hip import qwen_torch as qt

    cfg, layer, rope = _layer(64, 4, 2, seed=0)
    layer = layer.to(hip_device)
    cache = qt.build_qwen_torque_cache(bit_width=4, head_dim=64, kv_heads=2)
    adapter = qt.patch_vo_only_qwen_attention(layer, rotation=cache.torque_cache.rotation, cache=cache)
    x2 = torch.randn(2, 3, cfg.hidden_size, device=hip_device)
    cos, sin = rope(x2, torch.arange(3, device=hip_device)[None].expand(2, 3))
    with pytest.raises(ValueError, match="batch size 1"):
        adapter(x2, (cos, sin))
    x = torch.randn(1, 3, cfg.hidden_size, device=hip_device)
    cos, sin = rope(x, torch.arange(3, device=hip_device)[None])
    with torch.no_grad():
        adapter(x, (cos, sin))
        x1 = torch.randn(1, 1, cfg.hidden_size, device=hip_device)
        c1, s1 = rope(x1, torch.tensor([[3]], device=hip_device))
        adapter(x1, (c1, s1))
        with pytest.raises(RuntimeError, match="after switching to decode mode"):
            adapter(x, (cos, sin))
    q = torch.zeros(1, 4, 2, 64, device=hip_device)
    with pytest.raises(ValueError, match="q_len=1"):
        cache.decode_token(q)
    with pytest.raises(ValueError, match="single-token key/value"):
        cache.decode_token_with_current(q[:, :, :1], torch.zeros(1, 2, 2, 64, device=hip_device),
                                        torch.zeros(1, 2, 2, 64, device=hip_device))
    other = qt.build_qwen_torque_cache(bit_width=4, head_dim=64, kv_heads=2, rotation_seed=9)
    with pytest.raises(ValueError, match="rotation"):
        qt.TorqueQwenAttention(layer.self_attn.base_attn, rotation=cache.torque_cache.rotation, cache=other)

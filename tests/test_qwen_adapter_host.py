"""Host-side pieces of the Qwen attention adapter, on the CPU: the rotary embedding and the causal dense
attention of prompt chunks against transformers' own functions (qwen_mlx.py:819-848)."""

from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers.models.qwen3_next import modeling_qwen3_next as hf  # noqa: E402

from torque_hip import qwen_torch as qt  # noqa: E402


@pytest.mark.parametrize("head_dim,rotary_dim", [(64, 16), (128, 128), (256, 64)])
def test_rotary_matches_transformers(head_dim, rotary_dim):
    g = torch.Generator().manual_seed(head_dim)
    q = torch.randn(1, 4, 5, head_dim, generator=g)
    k = torch.randn(1, 2, 5, head_dim, generator=g)
    cos = torch.randn(1, 5, rotary_dim, generator=g)
    sin = torch.randn(1, 5, rotary_dim, generator=g)
    got = qt.apply_rotary(q, k, cos, sin)
    exp = hf.apply_rotary_pos_emb(q, k, cos, sin)
    for a, b in zip(got, exp):
        torch.testing.assert_close(a, b, atol=0, rtol=0)


@pytest.mark.parametrize("L,offset,group", [(7, 0, 2), (3, 5, 4), (1, 9, 1)])
def test_dense_chunk_attention_matches_eager(L, offset, group):
    g = torch.Generator().manual_seed(L + offset)
    hkv, d = 2, 64
    q = torch.randn(1, hkv * group, L, d, generator=g)
    k = torch.randn(1, hkv, offset + L, d, generator=g)
    v = torch.randn(1, hkv, offset + L, d, generator=g)
    got = qt._dense_attention(q, k, v, scale=d**-0.5, offset=offset)
    rows = torch.arange(offset, offset + L)[:, None]
    cols = torch.arange(offset + L)[None, :]
    mask = torch.where(cols <= rows, 0.0, float("-inf"))[None, None]
    module = torch.nn.Module()
    module.num_key_value_groups = group
    module.training = False
    exp, _ = hf.eager_attention_forward(module, q, k, v, mask, scaling=d**-0.5)
    torch.testing.assert_close(got, exp.transpose(1, 2), atol=2e-6, rtol=2e-5)

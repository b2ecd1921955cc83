"""Parity at the workload configurations of BASELINE.json, at their real sizes.

Synthetic inputs follow the configs: seeded fp16 N(0, std) Q/K/V, K scaled by
one log-normal(0, 1) factor per (layer, KV head, channel).  The oracle checks a
subset of KV heads / layers at the full sequence length (the oracle is a numpy
restatement; all heads at 32K-128K would take minutes), and size-independent
properties cover the rest: packed words bit-exact against the oracle packer,
decode invariant to the split count, and the tolerance of the north star
(max-abs 2e-3, relative L2 1e-3; observed values are ~1e-7).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import torque_oracle as o

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3
REL_L2 = 1e-3


def _close(got, exp, what):
    err = float(np.max(np.abs(got - exp)))
    rel = float(np.linalg.norm(got - exp) / np.linalg.norm(exp))
    assert err <= MAX_ABS and rel <= REL_L2, f"{what}: max-abs {err:.2e} rel-L2 {rel:.2e}"
    return err, rel


def _torch_synthetic(seed, layers, kv_heads, query_heads, seq_len, head_dim, std, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    q = (torch.randn((layers, query_heads, head_dim), generator=g, device=dev) * std).half()
    k = torch.randn((layers, kv_heads, seq_len, head_dim), generator=g, device=dev) * std
    v = (torch.randn((layers, kv_heads, seq_len, head_dim), generator=g, device=dev) * std).half()
    scale = torch.exp(torch.randn((layers, kv_heads, 1, head_dim), generator=g, device=dev))
    return q, (k * scale).half(), v


def _model(cache, layers=None, kv_heads=None):
    cfg = cache.config
    return o.OracleCache(
        bit_width=cfg.bit_width,
        head_dim=cfg.head_dim,
        num_layers=layers or cfg.num_layers,
        kv_heads=kv_heads or cfg.kv_heads,
        key_centroids=cache.key_codebook.centroids,
        value_centroids=cache.value_codebook.centroids,
        signs_left=cache.rotation.signs_left,
        signs_right=cache.rotation.signs_right,
        fused_weights=cfg.fused_weights,
    )


def _check_heads(cache, q, k, v, kv_subset, out):
    """Oracle on the chosen KV heads of layer 0 (with their query heads)."""
    cfg = cache.config
    group = q.shape[1] // cfg.kv_heads
    s = cache.sequence_length
    kc = cache._key_codes[:, :, :s].cpu().numpy().view(np.uint32)
    vc = cache._value_codes[:, :, :s].cpu().numpy().view(np.uint32)
    for kvh in kv_subset:
        model = _model(cache, layers=1, kv_heads=1)
        kk = k[:1, kvh : kvh + 1].float().cpu().numpy()
        vv = v[:1, kvh : kvh + 1].float().cpu().numpy()
        model.append(kk, vv)
        np.testing.assert_array_equal(kc[:1, kvh : kvh + 1], model.k_codes, err_msg=f"key codes head {kvh}")
        np.testing.assert_array_equal(vc[:1, kvh : kvh + 1], model.v_codes, err_msg=f"value codes head {kvh}")
        qh = q[:1, kvh * group : (kvh + 1) * group].float().cpu().numpy()
        _close(out[:1, kvh * group : (kvh + 1) * group], model.decode(qh), f"kv head {kvh}")


def _packed_cache(bits, head_dim, kv_heads, capacity, layers=1, seed=0):
    import torque_hip as th

    cfg = th.TorqueConfig(bit_width=bits, head_dim=head_dim, num_layers=layers, kv_heads=kv_heads, rotation_seed=seed)
    return th.TorqueKVCacheHIP(config=cfg, initial_capacity=capacity, decode_tail_capacity=0)


def test_c1_synthetic_512(hip_device):
    """C1: 512 tokens, D=128, 8 KV / 8 query heads, 4-bit -- every head against the oracle."""
    q, k, v = _torch_synthetic(1, 1, 8, 8, 512, 128, 1.0, hip_device)
    cache = _packed_cache(4, 128, 8, 512)
    cache.append_many(key=k, value=v)
    out = cache.decode(query=q, return_numpy=False).cpu().numpy()
    _check_heads(cache, q, k, v, range(8), out)


def test_c2_three_bit_decode_loop(hip_device):
    """C2: D=64, 3-bit (codes straddle words), 4 KV / 16 query heads, 4096 tokens then 64 one-token steps."""
    s0, steps = 4096, 64
    q, k, v = _torch_synthetic(2, 1, 4, 16, s0 + steps, 64, 1.0, hip_device)
    g = torch.Generator(device=hip_device).manual_seed(22)
    queries = torch.randn((steps, 1, 16, 64), generator=g, device=hip_device).half()
    cache = _packed_cache(3, 64, 4, 256)
    cache.append_many(key=k[:, :, :s0], value=v[:, :, :s0])
    model = _model(cache)
    model.append(k[:, :, :s0].float().cpu().numpy(), v[:, :, :s0].float().cpu().numpy())
    for step in range(steps):
        cache.append(key=k[:, :, s0 + step], value=v[:, :, s0 + step])
        out = cache.decode(query=queries[step], return_numpy=False)
        if step in (0, 31, 63):
            model.append(k[:, :, : s0 + step + 1].float().cpu().numpy()[:, :, model.sequence_length :],
                         v[:, :, : s0 + step + 1].float().cpu().numpy()[:, :, model.sequence_length :])
            _close(out.cpu().numpy(), model.decode(queries[step].float().cpu().numpy()), f"step {step}")
    kc = cache._key_codes[:, :, : s0 + steps].cpu().numpy().view(np.uint32)
    assert cache.sequence_length == s0 + steps and cache._store.capacity == 8192
    np.testing.assert_array_equal(kc[:, :, : model.sequence_length], model.k_codes)


@pytest.mark.parametrize("bits", [2, 4])
def test_c3_and_metric_shape_32k(hip_device, bits):
    """C3 (2-bit) and the metric shape M (4-bit): D=128, 8 KV / 32 query heads, 32768 tokens."""
    from torque_hip import ops

    q, k, v = _torch_synthetic(3 + bits, 1, 8, 32, 32768, 128, 1.0, hip_device)
    cache = _packed_cache(bits, 128, 8, 32768)
    cache.append_many(key=k, value=v)
    out = cache.decode(query=q, return_numpy=False).cpu().numpy()
    _check_heads(cache, q, k, v, (0, 5), out)
    store = cache._store
    for ns in (8, 17, 256):
        other = store.decode(q, rotate_query=True, inverse_output=True, n_splits=ns).cpu().numpy()
        np.testing.assert_allclose(other, out, atol=1e-6, rtol=1e-5, err_msg=f"n_splits {ns}")
    assert ops.plan_splits(1, 8, 32, 128, 32768, hip_device, bit_width=4) > 1


def test_c4_qwen_style_128k(hip_device):
    """C4: D=256, 4-bit, 2 KV / 8 query heads, 131072 tokens, std 0.5; plus the fp16-dense comparator."""
    from torque_hip import ops

    q, k, v = _torch_synthetic(4, 1, 2, 8, 131072, 256, 0.5, hip_device)
    cache = _packed_cache(4, 256, 2, 131072)
    cache.append_many(key=k, value=v)
    out = cache.decode(query=q, return_numpy=False).cpu().numpy()
    _check_heads(cache, q, k, v, (1,), out)
    dense = ops.dense_decode(q, k, v, num_layers=1, query_heads=8, kv_heads=2, head_dim=256, capacity=131072,
                             seq_len=131072).cpu().numpy()
    kk = k[0, 1].float().cpu().numpy()
    vv = v[0, 1].float().cpu().numpy()
    for qh in (4, 7):
        exp = o.attention_decode_dense(q[0, qh].float().cpu().numpy(), kk, vv)
        _close(dense[0, qh], exp, f"fp16-dense query head {qh}")


def test_c5_24_layer_decode_loop(hip_device):
    """C5: 24 layers, D=256, 4 KV / 16 query heads, 4-bit; prefill 8192 tokens, then 128 append+decode steps."""
    layers, s0, steps = 24, 8192, 128
    q, k, v = _torch_synthetic(5, layers, 4, 16, s0 + steps, 256, 1.0, hip_device)
    g = torch.Generator(device=hip_device).manual_seed(55)
    queries = torch.randn((steps, layers, 16, 256), generator=g, device=hip_device).half()
    cache = _packed_cache(4, 256, 4, s0 + steps, layers=layers)
    cache.append_many(key=k[:, :, :s0], value=v[:, :, :s0])
    outs = {}
    for step in range(steps):
        cache.append(key=k[:, :, s0 + step], value=v[:, :, s0 + step])
        out = cache.decode(query=queries[step], return_numpy=False)
        if step in (0, steps - 1):
            outs[step] = out.cpu().numpy()
    for step, out in outs.items():
        s = s0 + step + 1
        for layer in (0, 23):
            model = _model(cache, layers=1)
            model.append(k[layer : layer + 1, :, :s].float().cpu().numpy(), v[layer : layer + 1, :, :s].float().cpu().numpy())
            exp = model.decode(queries[step, layer : layer + 1].float().cpu().numpy())
            _close(out[layer : layer + 1], exp, f"step {step} layer {layer}")

"""GPU parity of the cache classes (TorqueKVCache, TorqueKVCacheHIP) against the oracle.

Mirrors tests/test_cache.py and tests/test_cache_mlx.py of the reference, plus
edge cases: empty and one-token caches, ragged lengths, capacity growth, GQA
group sizes 1/2/3/4/8, the rotation flags, fused_weights, float16 inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import torque_oracle as o

pytestmark = pytest.mark.gpu


def _uniform(bits):
    import torque_hip as th

    return th.build_uniform_codebook(bits)


def _oracle_for(cache, **kw):
    cfg = cache.config
    return o.OracleCache(
        bit_width=cfg.bit_width,
        head_dim=cfg.head_dim,
        num_layers=cfg.num_layers,
        kv_heads=cfg.kv_heads,
        key_centroids=cache.key_codebook.centroids,
        value_centroids=cache.value_codebook.centroids,
        signs_left=cache.rotation.signs_left,
        signs_right=cache.rotation.signs_right,
        fused_weights=cfg.fused_weights,
        **kw,
    )


def _codes(cache):
    s = cache.sequence_length
    return tuple(t[:, :, :s].cpu().numpy().view(np.uint32) for t in (cache._key_codes, cache._value_codes))


# ------------------------------------------------------------------ TorqueKVCache (reference cache.py API)


def test_cache_append_and_reset(hip_device):
    # test_cache.py:19-29
    import torque_hip as th

    cache = th.TorqueKVCache(config=th.TorqueConfig(bit_width=4, head_dim=64, num_layers=2, kv_heads=3),
                             key_codebook=_uniform(4), value_codebook=_uniform(4))
    payload = np.zeros((2, 3, 64), dtype=np.float32)
    cache.append(key=payload, value=payload)
    assert cache.sequence_length == 1
    cache.reset()
    assert cache.sequence_length == 0


def test_decode_single_token_matches_value(hip_device):
    # test_cache.py:32-46
    import torque_hip as th

    cache = th.TorqueKVCache(config=th.TorqueConfig(bit_width=4, head_dim=64), key_codebook=_uniform(4), value_codebook=_uniform(4))
    key = np.linspace(-1.0, 1.0, 64, dtype=np.float32)
    value = np.linspace(1.0, -1.0, 64, dtype=np.float32)
    cache.append(key=key, value=value)
    out = cache.decode(query=key.copy())
    _, values = cache.export_dequantized()
    np.testing.assert_allclose(out, cache.rotation.inverse(values[0, 0, 0]), rtol=1e-5, atol=1e-5)
    assert out.shape == (64,)


def test_metadata_variant(hip_device):
    # test_cache.py:49-57
    import torque_hip as th

    cache = th.TorqueKVCache(config=th.TorqueConfig(bit_width=3, head_dim=128, fused_weights=True),
                             key_codebook=_uniform(3), value_codebook=_uniform(3))
    assert cache.metadata.variant_id == "b3-h128-hadamard-fused"
    assert cache.metadata.codebook_name == "uniform"


def test_decode_shape_validation(hip_device):
    # test_cache.py:60-69
    import torque_hip as th

    cache = th.TorqueKVCache(config=th.TorqueConfig(bit_width=4, head_dim=64, num_layers=1, kv_heads=2),
                             key_codebook=_uniform(4), value_codebook=_uniform(4))
    payload = np.zeros((2, 64), dtype=np.float32)
    cache.append(key=payload, value=payload)
    with pytest.raises(ValueError):
        cache.decode(query=np.zeros((64,), dtype=np.float32))
    with pytest.raises(ValueError):
        cache.append(key=np.zeros((3, 64), np.float32), value=np.zeros((3, 64), np.float32))


def test_decode_matches_dequantized_reference(hip_device):
    # test_cache.py:72-94
    import torque_hip as th

    rng = np.random.default_rng(4)
    cache = th.TorqueKVCache(config=th.TorqueConfig(bit_width=4, head_dim=64), key_codebook=_uniform(4), value_codebook=_uniform(4))
    for _ in range(5):
        cache.append(key=rng.uniform(-1, 1, size=(64,)).astype(np.float32), value=rng.uniform(-1, 1, size=(64,)).astype(np.float32))
    query = rng.uniform(-1, 1, size=(64,)).astype(np.float32)
    out = cache.decode(query=query)
    keys, values = cache.export_dequantized()
    exp = o.rotation_inverse(
        o.streaming_attention_decode(o.rotation_apply(query, cache.rotation.signs_left, cache.rotation.signs_right), keys[0, 0], values[0, 0]),
        cache.rotation.signs_left, cache.rotation.signs_right,
    )
    np.testing.assert_allclose(out, exp, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(cache.decode_mlx(query=query), out, atol=1e-6)


def test_default_codebooks_and_build_cache(hip_device, tmp_path):
    """Gaussian defaults (seeds rs, rs+1) and TorqueArtifact.build_cache (artifact.py:157-162)."""
    import json

    import torque_hip as th
    from torque_hip.artifact import TorqueArtifact, TorqueArtifactManifest

    cfg = th.TorqueConfig(bit_width=4, head_dim=128, num_layers=2, kv_heads=2, fused_weights=True, rotation_seed=3)
    manifest = TorqueArtifactManifest(model_name="m", architecture="a", source_format="s", runtime_config=cfg,
                                      key_codebook=th.build_gaussian_codebook(4, seed=3),
                                      value_codebook=th.build_gaussian_codebook(4, seed=4))
    cache = TorqueArtifact(manifest=manifest).build_cache()
    assert isinstance(cache, th.TorqueKVCache) and cache.metadata.variant_id == "b4-h128-hadamard-fused"
    default = th.TorqueKVCache(config=cfg)
    np.testing.assert_array_equal(default.key_codebook.centroids, cache.key_codebook.centroids)
    np.testing.assert_array_equal(default.value_codebook.centroids, cache.value_codebook.centroids)
    rng = np.random.default_rng(0)
    model = _oracle_for(cache)
    for _ in range(40):
        k = rng.normal(size=(2, 2, 128)).astype(np.float32)
        v = rng.normal(size=(2, 2, 128)).astype(np.float32)
        cache.append(key=k, value=v)
        model.append(k[:, :, None], v[:, :, None])
    kc, vc = _codes(cache)
    np.testing.assert_array_equal(kc, model.k_codes)
    np.testing.assert_array_equal(vc, model.v_codes)
    q = rng.normal(size=(2, 2, 128)).astype(np.float32)
    np.testing.assert_allclose(cache.decode(query=q), model.decode(q), atol=1e-5, rtol=1e-5)


# ------------------------------------------------------------------ TorqueKVCacheHIP (reference cache_mlx.py API)


def test_capacity_growth(hip_device):
    # test_cache_mlx.py:21-34
    import torque_hip as th

    cache = th.TorqueKVCacheHIP(config=th.TorqueConfig(bit_width=4, head_dim=64, num_layers=2, kv_heads=2),
                                key_codebook=_uniform(4), value_codebook=_uniform(4), initial_capacity=2)
    rng = np.random.default_rng(1)
    model = _oracle_for(cache)
    for _ in range(5):
        k = rng.normal(size=(2, 2, 64)).astype(np.float32)
        cache.append(key=k, value=-k)
        model.append(k[:, :, None], -k[:, :, None])
    assert cache.sequence_length == 5 and cache.capacity >= 5 and cache._store.capacity == 8
    kc, vc = _codes(cache)
    np.testing.assert_array_equal(kc, model.k_codes)
    np.testing.assert_array_equal(vc, model.v_codes)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_append_many_bit_exact(hip_device, bits, head_dim, dtype):
    # test_cache_mlx.py:37-71 (exact equality of packed codes)
    import torque_hip as th

    rng = np.random.default_rng(3)
    cache = th.TorqueKVCacheHIP(config=th.TorqueConfig(bit_width=bits, head_dim=head_dim, num_layers=2, kv_heads=2),
                                key_codebook=th.build_gaussian_codebook(bits, seed=0),
                                value_codebook=th.build_gaussian_codebook(bits, seed=1), initial_capacity=8)
    keys = rng.normal(size=(2, 2, 37, head_dim)).astype(dtype)
    values = rng.normal(size=(2, 2, 37, head_dim)).astype(dtype)
    cache.append_many(key=keys, value=values)
    model = _oracle_for(cache)
    model.append(keys.astype(np.float32), values.astype(np.float32))
    kc, vc = _codes(cache)
    np.testing.assert_array_equal(kc, model.k_codes)
    np.testing.assert_array_equal(vc, model.v_codes)
    # argmin (the numpy cache's quantizer) agrees on these inputs too
    rot = o.rotation_apply(keys.astype(np.float32), cache.rotation.signs_left, cache.rotation.signs_right)
    np.testing.assert_array_equal(kc, o.pack_indices_batched(o.quantize_argmin(rot, cache.key_codebook.centroids), bits))
    assert cache.sequence_length == 37


@pytest.mark.parametrize("group", [1, 2, 3, 4, 8])
def test_grouped_decode_matches_reference(hip_device, group):
    # test_cache_mlx.py:74-116 (reference group 2); kv = q // group
    import torque_hip as th

    rng = np.random.default_rng(9)
    cfg = th.TorqueConfig(bit_width=4, head_dim=64, num_layers=1, kv_heads=2)
    cache = th.TorqueKVCacheHIP(config=cfg, key_codebook=_uniform(4), value_codebook=_uniform(4), initial_capacity=8)
    model = _oracle_for(cache)
    for _ in range(6):
        k = rng.uniform(-1, 1, size=(2, 64)).astype(np.float32)
        v = rng.uniform(-1, 1, size=(2, 64)).astype(np.float32)
        cache.append(key=k, value=v)
        model.append(k[None, :, None], v[None, :, None])
    q = rng.uniform(-1, 1, size=(2 * group, 64)).astype(np.float32)
    got = cache.decode(query=q)
    assert got.shape == (2 * group, 64)
    np.testing.assert_allclose(got, model.decode(q[None])[0], atol=1e-5, rtol=1e-5)
    keys, values = cache.export_dequantized()
    for h in range(2 * group):
        out_rot = o.streaming_attention_decode(o.rotation_apply(q[h], model.signs_left, model.signs_right), keys[0, h // group], values[0, h // group])
        np.testing.assert_allclose(got[h], o.rotation_inverse(out_rot, model.signs_left, model.signs_right), atol=1e-5)


@pytest.mark.parametrize("tail", [0, 2])
def test_decode_with_current_equals_append_then_decode(hip_device, tail):
    # test_cache_mlx.py:165-208
    import torque_hip as th

    rng = np.random.default_rng(23)
    cfg = th.TorqueConfig(bit_width=4, head_dim=64, num_layers=1, kv_heads=2)
    a = th.TorqueKVCacheHIP(config=cfg, key_codebook=_uniform(4), value_codebook=_uniform(4), initial_capacity=8, decode_tail_capacity=tail)
    b = th.TorqueKVCacheHIP(config=cfg, key_codebook=_uniform(4), value_codebook=_uniform(4), initial_capacity=8, decode_tail_capacity=tail)
    for _ in range(4):
        k = rng.uniform(-1, 1, size=(2, 64)).astype(np.float32)
        v = rng.uniform(-1, 1, size=(2, 64)).astype(np.float32)
        a.append(key=k, value=v)
        b.append(key=k, value=v)
    q = rng.uniform(-1, 1, size=(4, 64)).astype(np.float32)
    ck = rng.uniform(-1, 1, size=(2, 64)).astype(np.float32)
    cv = rng.uniform(-1, 1, size=(2, 64)).astype(np.float32)
    got = a.decode_mlx_with_current(query=q, key=ck, value=cv)
    b.append(key=ck, value=cv)
    np.testing.assert_allclose(got, b.decode_mlx(query=q), atol=1e-5, rtol=1e-5)
    assert a.sequence_length == 4


def test_decode_with_current_on_empty_cache(hip_device):
    import torque_hip as th

    rng = np.random.default_rng(2)
    cfg = th.TorqueConfig(bit_width=3, head_dim=128, num_layers=1, kv_heads=1)
    cache = th.TorqueKVCacheHIP(config=cfg, key_codebook=_uniform(3), value_codebook=_uniform(3))
    ck = rng.normal(size=(128,)).astype(np.float32)
    cv = rng.normal(size=(128,)).astype(np.float32)
    got = cache.decode_with_current(query=rng.normal(size=(128,)).astype(np.float32), key=ck, value=cv)
    model = _oracle_for(cache)
    model.append(ck.reshape(1, 1, 1, 128), cv.reshape(1, 1, 1, 128))
    _, values = model.export_dequantized()
    np.testing.assert_allclose(got, o.rotation_inverse(values[0, 0, 0], model.signs_left, model.signs_right), atol=1e-5)


def test_strategies(hip_device):
    # test_cache_mlx.py:211-236 plus agreement of every strategy
    import torque_hip as th

    rng = np.random.default_rng(5)
    cfg = th.TorqueConfig(bit_width=4, head_dim=128, num_layers=2, kv_heads=2)
    caches = {s: th.TorqueKVCacheHIP(config=cfg, key_codebook=_uniform(4), value_codebook=_uniform(4), decode_strategy=s)
              for s in th.SUPPORTED_DECODE_STRATEGIES}
    assert caches["auto"].resolve_decode_strategy(sequence_length=128) == "split_batched"
    assert caches["split_batched"].resolve_decode_strategy(sequence_length=32) == "split_batched"
    k = rng.normal(size=(2, 2, 3000, 128)).astype(np.float32)
    v = rng.normal(size=(2, 2, 3000, 128)).astype(np.float32)
    q = rng.normal(size=(2, 8, 128)).astype(np.float32)
    outs = {}
    for s, c in caches.items():
        c.append_many(key=k, value=v)
        outs[s] = c.decode(query=q)
    profiled = th.TorqueKVCacheHIP(config=cfg, key_codebook=_uniform(4), value_codebook=_uniform(4), profile_decode_components=True)
    profiled.append_many(key=k, value=v)
    outs["profiled"] = profiled.decode(query=q)
    assert {"packed_score_seconds", "softmax_seconds", "packed_value_seconds"} <= set(profiled.last_decode_profile)
    model = _oracle_for(caches["auto"])
    model.append(k, v)
    exp = model.decode(q)
    for s, out in outs.items():
        np.testing.assert_allclose(out, exp, atol=2e-5, rtol=1e-4, err_msg=s)


@pytest.mark.parametrize("prefill", [0, 1, 700])
def test_profiled_decode_with_current_and_decode_append(hip_device, prefill):
    """profile_decode_components on decode_with_current and decode_append runs the reference's staged
    path with the current token (cache_mlx.py:565-640) and records its stage keys, including
    tail_seconds; outputs (and, for decode_append, packed words and length) equal the unprofiled calls."""
    import torque_hip as th

    rng = np.random.default_rng(prefill + 3)
    cfg = th.TorqueConfig(bit_width=4, head_dim=128, num_layers=2, kv_heads=2)
    kw = dict(config=cfg, key_codebook=th.build_gaussian_codebook(4, seed=0),
              value_codebook=th.build_gaussian_codebook(4, seed=1), initial_capacity=8)
    plain, profiled = th.TorqueKVCacheHIP(**kw), th.TorqueKVCacheHIP(**kw, profile_decode_components=True)
    if prefill:
        k0 = rng.normal(size=(2, 2, prefill, 128)).astype(np.float32)
        v0 = rng.normal(size=(2, 2, prefill, 128)).astype(np.float32)
        plain.append_many(key=k0, value=v0)
        profiled.append_many(key=k0, value=v0)
    stage_keys = {"packed_score_seconds", "softmax_seconds", "packed_value_seconds", "tail_seconds"}
    for step in range(3):
        q = rng.normal(size=(2, 8, 128)).astype(np.float32)
        k = rng.normal(size=(2, 2, 128)).astype(np.float32)
        v = rng.normal(size=(2, 2, 128)).astype(np.float32)
        exp = plain.decode_with_current(query=q, key=k, value=v)
        got = profiled.decode_with_current(query=q, key=k, value=v)
        np.testing.assert_allclose(got, exp, atol=2e-6, rtol=1e-5, err_msg=f"with_current step {step}")
        keys = set(profiled.last_decode_profile)
        assert (stage_keys if plain.sequence_length else {"tail_seconds"}) <= keys, keys
        exp = plain.decode_append(query=q, key=k, value=v)
        got = profiled.decode_append(query=q, key=k, value=v)
        np.testing.assert_allclose(got, exp, atol=2e-6, rtol=1e-5, err_msg=f"decode_append step {step}")
        assert "append_seconds" in profiled.last_decode_profile
        assert profiled.sequence_length == plain.sequence_length == prefill + step + 1
        s = plain.sequence_length
        for a, b in ((plain._key_codes, profiled._key_codes), (plain._value_codes, profiled._value_codes)):
            np.testing.assert_array_equal(a[:, :, :s].cpu().numpy(), b[:, :, :s].cpu().numpy())
    assert all(t >= 0.0 for t in profiled.last_decode_profile.values())


@pytest.mark.parametrize("seq_len", [1, 7, 255, 256, 257, 1000, 4097])
def test_ragged_lengths_and_split_invariance(hip_device, seq_len):
    import torque_hip as th
    from torque_hip import ops

    rng = np.random.default_rng(seq_len)
    cfg = th.TorqueConfig(bit_width=4, head_dim=128, num_layers=1, kv_heads=4)
    cache = th.TorqueKVCacheHIP(config=cfg, key_codebook=th.build_gaussian_codebook(4, seed=0),
                                value_codebook=th.build_gaussian_codebook(4, seed=1), initial_capacity=16)
    k = rng.normal(size=(1, 4, seq_len, 128)).astype(np.float16)
    v = rng.normal(size=(1, 4, seq_len, 128)).astype(np.float16)
    q = rng.normal(size=(1, 16, 128)).astype(np.float16)
    cache.append_many(key=k, value=v)
    model = _oracle_for(cache)
    model.append(k.astype(np.float32), v.astype(np.float32))
    exp = model.decode(q.astype(np.float32))
    store = cache._store
    qd = torch.from_numpy(q).to(hip_device)
    for n_splits in (None, 1, 3, 64, 256):
        got = store.decode(qd, rotate_query=True, inverse_output=True, n_splits=n_splits).cpu().numpy()
        np.testing.assert_allclose(got, exp, atol=2e-5, rtol=1e-4, err_msg=f"n_splits={n_splits}")
    assert ops.plan_splits(1, 4, 16, 128, seq_len, hip_device) >= 1


def test_flags_and_fused_weights(hip_device):
    """rotate_*_on_append / rotate_queries_on_decode (cache_mlx.py:52-54) and fused_weights (cache.py:131-134)."""
    import torque_hip as th

    rng = np.random.default_rng(11)
    k = rng.normal(size=(2, 2, 50, 64)).astype(np.float32)
    v = rng.normal(size=(2, 2, 50, 64)).astype(np.float32)
    q = rng.normal(size=(2, 4, 64)).astype(np.float32)
    for fused in (False, True):
        for rk, rv, rq in ((True, True, True), (True, False, True), (False, False, False), (True, True, False)):
            cfg = th.TorqueConfig(bit_width=4, head_dim=64, num_layers=2, kv_heads=2, fused_weights=fused)
            cache = th.TorqueKVCacheHIP(config=cfg, key_codebook=_uniform(4), value_codebook=_uniform(4),
                                        rotate_keys_on_append=rk, rotate_values_on_append=rv, rotate_queries_on_decode=rq)
            cache.append_many(key=k, value=v)
            model = _oracle_for(cache, rotate_keys_on_append=rk, rotate_values_on_append=rv, rotate_queries_on_decode=rq)
            model.append(k, v)
            kc, vc = _codes(cache)
            np.testing.assert_array_equal(kc, model.k_codes)
            np.testing.assert_array_equal(vc, model.v_codes)
            np.testing.assert_allclose(cache.decode(query=q), model.decode(q), atol=1e-5, rtol=1e-5)


def test_shape_forms_and_errors(hip_device):
    """Input forms of cache_mlx.py:442-466, 724-740 and output squeezing (cache_mlx.py:340-351)."""
    import torque_hip as th

    one = th.TorqueKVCacheHIP(config=th.TorqueConfig(bit_width=4, head_dim=64), key_codebook=_uniform(4), value_codebook=_uniform(4))
    assert one.decode(query=np.ones(64, np.float32)).shape == (64,)  # empty cache -> zeros
    assert not one.decode(query=np.ones(64, np.float32)).any()
    one.append(key=np.ones(64, np.float32), value=np.ones(64, np.float32))
    one.append_many(key=np.ones((1, 5, 64), np.float32), value=np.ones((1, 5, 64), np.float32))  # [Hkv, S, D]
    assert one.sequence_length == 6 and one.offset == 6
    two = th.TorqueKVCacheHIP(config=th.TorqueConfig(bit_width=4, head_dim=64, num_layers=2, kv_heads=2),
                              key_codebook=_uniform(4), value_codebook=_uniform(4))
    with pytest.raises(ValueError, match="only valid for 1 layer"):
        two.append(key=np.ones((2, 64), np.float32), value=np.ones((2, 64), np.float32))
    with pytest.raises(ValueError, match="must have shape"):
        two.append(key=np.ones((2, 3, 64), np.float32), value=np.ones((2, 3, 64), np.float32))
    with pytest.raises(ValueError, match="key/value sequence dimensions must match"):
        two.append_many(key=np.ones((2, 2, 3, 64), np.float32), value=np.ones((2, 2, 4, 64), np.float32))
    two.append(key=np.ones((2, 2, 64), np.float32), value=np.ones((2, 2, 64), np.float32))
    with pytest.raises(ValueError, match="must be divisible by kv_heads"):
        two.decode(query=np.ones((2, 3, 64), np.float32))
    with pytest.raises(ValueError, match="single current token"):
        two.decode_with_current(query=np.ones((2, 2, 64), np.float32), key=np.ones((2, 2, 2, 64), np.float32),
                                value=np.ones((2, 2, 2, 64), np.float32))
    out = two.decode(query=np.ones((2, 4, 64), np.float32), return_numpy=False)
    assert isinstance(out, torch.Tensor) and out.is_cuda and tuple(out.shape) == (2, 4, 64)
    assert two.make_mask(1) is None and two.make_mask(3) == "causal"
    mask = two.make_mask(3, return_array=True)
    assert tuple(mask.shape) == (3, 4) and bool(mask[0, 0]) and not bool(mask[0, 2])
    two.reset()
    assert two.sequence_length == 0 and not two._store.key_codes.any().item()


def test_split_merge_handoff_is_coherent(hip_device):
    """Many-split decodes hand partials between workgroups through one shared
    workspace; alternate two caches so a stale partial from the previous call
    would show up.  Single-split decodes need no hand-off and are the check."""
    import torque_hip as th

    rng = np.random.default_rng(77)
    caches, queries = [], []
    for seed, s in ((0, 20000), (1, 9000)):
        cfg = th.TorqueConfig(bit_width=4, head_dim=128, num_layers=1, kv_heads=8, rotation_seed=seed)
        c = th.TorqueKVCacheHIP(config=cfg, initial_capacity=s)
        c.append_many(key=rng.normal(size=(1, 8, s, 128)).astype(np.float16),
                      value=rng.normal(size=(1, 8, s, 128)).astype(np.float16))
        caches.append(c)
        queries.append(torch.from_numpy(rng.normal(size=(1, 32, 128)).astype(np.float32)).to(hip_device))
    refs = [c._store.decode(q, rotate_query=True, inverse_output=True, n_splits=1).cpu().numpy()
            for c, q in zip(caches, queries)]
    for rep in range(40):
        i = rep % 2
        ns = (16, 64, 256, 37)[rep % 4]
        got = caches[i]._store.decode(queries[i], rotate_query=True, inverse_output=True, n_splits=ns).cpu().numpy()
        np.testing.assert_allclose(got, refs[i], atol=2e-6, rtol=1e-5, err_msg=f"rep {rep} cache {i} n_splits {ns}")

"""Per-vector scales on the GPU (``scale_mode="rms"``).

An opt-in extension with no reference counterpart: the reference's codes index
one global codebook per stream (quantization.py:120-148).  Pinned as follows:
the codes equal the reference's boundary-count quantizer and packer
(quantization.py:139-148, 176-201) applied to rot(x) / s with the kernel's own
scales s (bit-exact); the scales equal the oracle RMS of rot(x) up to the
float32 rounding of the sum; dequantization and decode are checked against the
oracle on those codes and scales; the dequantizing, packing and decode-append
paths agree exactly with one another; and on rows whose norms vary the scaled
cache tracks unquantized attention more closely than the unscaled one.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import torque_oracle as o

pytestmark = pytest.mark.gpu


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _varied_rows(rng, shape, spread=2.0):
    """N(0, 1) rows times a log-normal per-row gain (norms over a few decades)."""
    x = rng.normal(size=shape) * rng.lognormal(0.0, spread, size=shape[:-1] + (1,))
    return x.astype(np.float16)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
def test_append_scaled_codes_and_scales(hip_device, bits, head_dim):
    from torque_hip import _lib

    L, H, S, offset, cap = 2, 3, 37, 5, 50
    W = o.packed_words_for_head_dim(head_dim, bits)
    rng = np.random.default_rng(bits * 1000 + head_dim)
    keys = _varied_rows(rng, (L, H, S, head_dim))
    values = _varied_rows(rng, (L, H, S, head_dim))
    keys[1, 2, 7] = 0.0  # an all-zero row keeps scale 1
    sl, sr = o.rotation_signs_from_seed(head_dim, 2)
    kcb, vcb = o.build_gaussian_codebook(bits, seed=1), o.build_gaussian_codebook(bits, seed=2)
    kb, vb = o.codebook_boundaries(kcb), o.codebook_boundaries(vcb)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(hip_device)  # noqa: E731
    kc = torch.zeros(L, H, cap, W, dtype=torch.int32, device=hip_device)
    vc = torch.zeros_like(kc)
    ks = torch.zeros(L, H, cap, dtype=torch.float32, device=hip_device)
    vs = torch.zeros_like(ks)
    tk, tv, tsl, tsr, tkb, tvb = d(keys), d(values), d(sl), d(sr), d(kb), d(vb)
    _lib.call("tq_append_scaled", tk.data_ptr(), tv.data_ptr(), _lib.TQ_F16, L, H, S, head_dim, bits, tsl.data_ptr(),
              tsr.data_ptr(), _lib.TQ_ROTATE_KEYS | _lib.TQ_ROTATE_VALUES, tkb.data_ptr(), tvb.data_ptr(),
              kc.data_ptr(), vc.data_ptr(), ks.data_ptr(), vs.data_ptr(), cap, offset, _stream())
    torch.cuda.synchronize()
    for x, codes, scales, bnd in ((keys, kc, ks, kb), (values, vc, vs, vb)):
        rot = o.rotation_apply(x.astype(np.float32), sl, sr)
        got_s = scales[:, :, offset : offset + S].cpu().numpy()
        np.testing.assert_allclose(got_s, o.rms_scales(rot), rtol=3e-6)
        exp_codes, _ = o.quantize_scaled(rot, bnd, got_s)
        exp = o.pack_indices_batched(exp_codes.reshape(-1, head_dim), bits).reshape(L, H, S, W)
        np.testing.assert_array_equal(codes[:, :, offset : offset + S].cpu().numpy().view(np.uint32), exp)
        assert not scales[:, :, :offset].any() and not scales[:, :, offset + S :].any()
    assert float(ks[1, 2, offset + 7]) == 1.0


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_scaled_dequantize_unpack_and_pack_paths_agree(hip_device, bits):
    """tq_quantize_dequantize_scaled == tq_unpack_dequantize_scaled of tq_append_scaled, bit for bit,
    and both equal centroid(code) x scale from the oracle on the kernel's codes and scales."""
    from torque_hip import _lib

    L, H, D = 2, 4, 128
    W = o.packed_words_for_head_dim(D, bits)
    rng = np.random.default_rng(31 + bits)
    x = torch.from_numpy(_varied_rows(rng, (L, H, 1, D))).to(hip_device)
    y = torch.from_numpy(_varied_rows(rng, (L, H, 1, D))).to(hip_device)
    sl, sr = o.rotation_signs_from_seed(D, 4)
    kcb, vcb = o.build_gaussian_codebook(bits, seed=3), o.build_gaussian_codebook(bits, seed=4)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(hip_device)  # noqa: E731
    tsl, tsr = t(sl), t(sr)
    kb, vb, kcent, vcent = t(o.codebook_boundaries(kcb)), t(o.codebook_boundaries(vcb)), t(kcb), t(vcb)
    flags = _lib.TQ_ROTATE_KEYS | _lib.TQ_ROTATE_VALUES
    kq = torch.empty(L, H, D, dtype=torch.float32, device=hip_device)
    vq = torch.empty_like(kq)
    _lib.call("tq_quantize_dequantize_scaled", x.data_ptr(), y.data_ptr(), _lib.TQ_F16, L * H, D, bits,
              tsl.data_ptr(), tsr.data_ptr(), flags, kb.data_ptr(), vb.data_ptr(), kcent.data_ptr(),
              vcent.data_ptr(), kq.data_ptr(), vq.data_ptr(), _stream())
    kc = torch.zeros(L, H, 1, W, dtype=torch.int32, device=hip_device)
    vc = torch.zeros_like(kc)
    ks = torch.zeros(L, H, 1, dtype=torch.float32, device=hip_device)
    vs = torch.zeros_like(ks)
    _lib.call("tq_append_scaled", x.data_ptr(), y.data_ptr(), _lib.TQ_F16, L, H, 1, D, bits, tsl.data_ptr(),
              tsr.data_ptr(), flags, kb.data_ptr(), vb.data_ptr(), kc.data_ptr(), vc.data_ptr(), ks.data_ptr(),
              vs.data_ptr(), 1, 0, _stream())
    for codes, scales, cent, q in ((kc, ks, kcent, kq), (vc, vs, vcent, vq)):
        out = torch.empty(L, H, 1, D, dtype=torch.float32, device=hip_device)
        _lib.call("tq_unpack_dequantize_scaled", codes.data_ptr(), scales.data_ptr(), L * H, 1, 1, D, bits,
                  cent.data_ptr(), out.data_ptr(), _stream())
        torch.cuda.synchronize()
        assert torch.equal(out[:, :, 0], q)
        idx = o.unpack_indices_batched(codes.cpu().numpy().view(np.uint32).reshape(-1, W), bits, D)
        exp = o.dequantize_scaled(idx, cent.cpu().numpy(), scales.cpu().numpy().reshape(-1))
        np.testing.assert_array_equal(out.cpu().numpy().reshape(-1, D), exp)


def _expected_decode(cache, q):
    """Oracle decode over the cache's own dequantized contents (codes x scales), rotated basis."""
    keys, values = cache.export_dequantized()
    sl, sr = cache.rotation.signs_left, cache.rotation.signs_right
    cfg = cache.config
    hq = q.shape[1]
    g = hq // cfg.kv_heads
    out = np.zeros((cfg.num_layers, hq, cfg.head_dim), dtype=np.float64)
    for layer in range(cfg.num_layers):
        for h in range(hq):
            qr = o.rotation_apply(q[layer, h].astype(np.float32), sl, sr)
            r = o.attention_decode_dense(qr, keys[layer, h // g], values[layer, h // g])
            out[layer, h] = r if cfg.fused_weights else o.rotation_inverse(r.astype(np.float32), sl, sr)
    return out


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize(("head_dim", "kv_heads", "query_heads"), [(64, 2, 2), (128, 2, 8), (256, 1, 4)])
@pytest.mark.parametrize("strategy", ["split_batched", "fused_per_head"])
def test_rms_cache_decode_matches_oracle(hip_device, bits, head_dim, kv_heads, query_heads, strategy):
    import torque_hip as th

    cfg = th.TorqueConfig(bit_width=bits, head_dim=head_dim, num_layers=2, kv_heads=kv_heads, scale_mode="rms")
    assert cfg.variant_id.endswith("-rms")
    cache = th.TorqueKVCacheHIP(config=cfg, initial_capacity=64, decode_strategy=strategy)
    rng = np.random.default_rng(bits + head_dim)
    for n in (150, 1, 37):  # prefill, a single token, a ragged chunk; capacity grows 64 -> 256
        cache.append_many(key=_varied_rows(rng, (2, kv_heads, n, head_dim)),
                          value=_varied_rows(rng, (2, kv_heads, n, head_dim)))
    assert cache.sequence_length == 188 and cache._store.capacity == 256
    q = rng.normal(size=(2, query_heads, head_dim)).astype(np.float32)
    got = cache.decode(query=q)
    exp = _expected_decode(cache, q)
    # Row gains span ~e^(+-6): fp32 accumulation error is relative to the output's magnitude.
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5 * float(np.abs(exp).max()))
    assert np.linalg.norm(got - exp) <= 1e-5 * np.linalg.norm(exp)


def test_rms_cache_with_current_and_decode_append(hip_device):
    import torque_hip as th

    cfg = th.TorqueConfig(bit_width=4, head_dim=128, num_layers=2, kv_heads=2, scale_mode="rms")
    rng = np.random.default_rng(8)
    prefill = [_varied_rows(rng, (2, 2, 300, 128)) for _ in range(2)]
    caches = [th.TorqueKVCacheHIP(config=cfg, initial_capacity=512) for _ in range(3)]
    for c in caches:
        c.append_many(key=prefill[0], value=prefill[1])
    for _ in range(3):
        q = rng.normal(size=(2, 8, 128)).astype(np.float16)
        k, v = _varied_rows(rng, (2, 2, 128)), _varied_rows(rng, (2, 2, 128))
        with_cur = caches[0].decode_with_current(query=q, key=k, value=v)
        caches[0].append(key=k, value=v)
        fused = caches[1].decode_append(query=q, key=k, value=v)
        caches[2].append(key=k, value=v)
        after = caches[2].decode(query=q)
        np.testing.assert_array_equal(fused, with_cur)
        np.testing.assert_allclose(after, with_cur, atol=2e-6, rtol=1e-5)
    for a, b in ((caches[0], caches[1]), (caches[0], caches[2])):
        s = a.sequence_length
        assert b.sequence_length == s
        for name in ("key_codes", "value_codes", "key_scales", "value_scales"):
            assert torch.equal(getattr(a._store, name)[:, :, :s], getattr(b._store, name)[:, :, :s]), name


def test_rms_mode_tracks_unquantized_attention_better(hip_device):
    """Rows whose norms span decades: the scaled cache's decode is closer to attention over the unquantized
    rows than the unscaled cache's (the point of per-vector scales)."""
    import torque_hip as th

    rng = np.random.default_rng(12)
    keys = _varied_rows(rng, (1, 2, 512, 128), spread=1.5)
    values = _varied_rows(rng, (1, 2, 512, 128), spread=1.5)
    q = (rng.normal(size=(1, 8, 128)) * 0.05).astype(np.float32)
    exact = np.stack([
        o.attention_decode_dense(q[0, h], keys[0, h // 4].astype(np.float32), values[0, h // 4].astype(np.float32))
        for h in range(8)
    ])[None]
    errs = {}
    for mode in ("none", "rms"):
        cache = th.TorqueKVCacheHIP(config=th.TorqueConfig(bit_width=4, head_dim=128, kv_heads=2, scale_mode=mode),
                                    initial_capacity=512)
        cache.append_many(key=keys, value=values)
        got = cache.decode(query=q).reshape(exact.shape)
        errs[mode] = float(np.linalg.norm(got - exact) / np.linalg.norm(exact))
    assert errs["rms"] < 0.5 * errs["none"], errs


def test_rms_manifest_builds_scaled_cache(hip_device):
    """A manifest whose runtime_config carries scale_mode "rms" survives JSON and builds a scaled
    TorqueKVCache (the reference cache.py API) whose decode matches the oracle on its own contents."""
    import json

    import torque_hip as th
    from torque_hip.artifact import TorqueArtifact, TorqueArtifactManifest

    cfg = th.TorqueConfig(bit_width=3, head_dim=64, num_layers=2, kv_heads=2, fused_weights=True, rotation_seed=5,
                          scale_mode="rms")
    manifest = TorqueArtifactManifest(model_name="m", architecture="a", source_format="s", runtime_config=cfg,
                                      key_codebook=th.build_gaussian_codebook(3, seed=5),
                                      value_codebook=th.build_gaussian_codebook(3, seed=6))
    manifest = TorqueArtifactManifest.from_dict(json.loads(json.dumps(manifest.to_dict())))
    assert manifest.runtime_config.scale_mode == "rms"
    cache = TorqueArtifact(manifest=manifest).build_cache()
    assert isinstance(cache, th.TorqueKVCache) and cache.metadata.variant_id == "b3-h64-hadamard-fused-rms"
    rng = np.random.default_rng(21)
    for _ in range(30):
        cache.append(key=_varied_rows(rng, (2, 2, 64)).astype(np.float32),
                     value=_varied_rows(rng, (2, 2, 64)).astype(np.float32))
    assert cache._store.scaled and bool((cache._store.key_scales[:, :, :30] > 0).all())
    q = rng.normal(size=(2, 2, 64)).astype(np.float32)
    got = cache.decode(query=q)
    exp = _expected_decode(cache, q)
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5 * float(np.abs(exp).max()))
